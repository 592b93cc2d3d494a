"""CPU tests of the oracle (the C restatement under oracle/): pinned against the expected values the
reference's own tests hold (tests/golden/reference_vectors.json), against exact-arithmetic restatements of the
summation orders it documents, and against closed forms and brute-force integer sums. No GPU is used here."""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "reference_vectors.json")))
Q8, Q4, Q4K, Q6K = 1, 2, 3, 4
DTS = (Q8, Q4, Q4K, Q6K)
BLOCK = O.BLOCK


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- exact float32 arithmetic (for order pins)
def rne32(v):
    """Round an exact rational to the nearest float32 (ties to even, subnormals kept); returns np.float32."""
    v = Fraction(v)
    if v == 0:
        return np.float32(0.0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    n = m.numerator // m.denominator
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(n * ulp))


def fma32(a, b, c):
    return rne32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def add32(a, b):
    return rne32(Fraction(float(a)) + Fraction(float(b)))


def sdot32_exact(x, y):
    """cpu_gemv_amd64.s:69-106: element i is fused into chain i mod 32 (register (i/8) mod 4, lane i mod 8) in
    ascending i; Y[l] = (A0+A1)+(A2+A3), s_l = Y[l]+Y[l+4], result = (s0+s2)+(s1+s3)."""
    acc = [np.float32(0.0)] * 32
    for i in range(len(x)):
        acc[i % 32] = fma32(x[i], y[i], acc[i % 32])
    Y = [add32(add32(acc[l], acc[8 + l]), add32(acc[16 + l], acc[24 + l])) for l in range(8)]
    s = [add32(Y[l], Y[l + 4]) for l in range(4)]
    return add32(add32(s[0], s[2]), add32(s[1], s[3]))


# ---------------------------------------------------------------- dequantization (a1-a8)
@pytest.mark.parametrize("case", GOLD["dequant_golden"]["cases"], ids=lambda c: "dt%d" % c["dtype"])
def test_dequant_matches_reference_golden(case):
    """FNV-1a-64 of the dequantized float32 bits and one sample, as TestDequantMatchesLlamaCpp holds them."""
    raw = O.random_quant(case["dtype"], case["seed"], GOLD["dequant_golden"]["blocks"])
    y = O.dequant(case["dtype"], raw)
    assert "%016x" % O.fnv(y) == case["fnv1a64"]
    assert "%08x" % int(y.view(np.uint32)[case["at"]]) == case["bits"]


@pytest.mark.parametrize("case", GOLD["dequant_known"]["cases"], ids=lambda c: "dt%d" % c["dtype"])
def test_dequant_known_values(case):
    raw = np.zeros(BLOCK[case["dtype"]][1], np.uint8)
    for k, v in case["set"].items():
        raw[int(k)] = v
    y = O.dequant(case["dtype"], raw)
    for k, v in case["expect"].items():
        assert y[int(k)] == np.float32(v), (k, y[int(k)], v)


def test_zero_raw_q4_is_plus_zero():
    g = GOLD["zero_raw_q4"]
    raw = O.quant_zero_raw(Q4, g["blocks"] * 32)
    for k, v in g["byte_expect"].items():
        assert raw[int(k)] == v
    assert np.all(O.dequant(Q4, raw).view(np.uint32) == 0)


@pytest.mark.parametrize("dt", DTS)
def test_zero_raw_all_dtypes_open_to_zero(dt):
    """QuantZeroRaw (quant.go:416-427): all bytes 0 except q4's codes. q6_k opens to fl(0*sc)*(0-32) = -0,
    which the reference accepts (quant.go:408-409); only q4 needs its codes moved to keep +0."""
    raw = O.quant_zero_raw(dt, 2 * BLOCK[dt][0])
    y = O.dequant(dt, raw)
    assert np.all(y == 0)
    if dt != Q6K:
        assert np.all(y.view(np.uint32) == 0)


@pytest.mark.parametrize("dt", DTS)
def test_zero_scale_gives_zero(dt):
    g = GOLD["zero_scale"]
    raw = np.full(BLOCK[dt][1], g["fill"], np.uint8)
    for i in g["zero_bytes"][str(dt)]:
        raw[i] = 0
    assert np.all(O.dequant(dt, raw) == 0)


@pytest.mark.parametrize("case", GOLD["check_scales"]["cases"], ids=lambda c: "dt%d+%d" % (c["dtype"], c["at"]))
def test_check_quant_scales(case):
    dt, at = case["dtype"], case["at"]
    size = BLOCK[dt][1]
    assert O.check_quant_scales(dt, np.zeros(3 * size, np.uint8)) == -1
    for bad in GOLD["check_scales"]["bad_values"]:
        raw = np.zeros(3 * size, np.uint8)
        raw[size + at] = bad & 0xFF
        raw[size + at + 1] = bad >> 8
        assert O.check_quant_scales(dt, raw) == 1


def test_f16_subnormal_and_nan_payload():
    """f16ToF32 (cpu_dtype.go:126-145) is exact: every finite half maps to its value, NaN payloads are kept."""
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    got = np.array([O.lib().trq_f16_to_f32(int(v)) for v in h[::97]], np.float32)
    want = h[::97].view(np.float16).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))


# ---------------------------------------------------------------- fp32 dot order (a9, a10)
@pytest.mark.parametrize("K", [32, 64, 96])
def test_dot_f32_follows_sdot32_order_exactly(K):
    """The oracle's dot equals an exact-rational restatement of the sdot32 chains and tree. Inputs span many
    magnitudes so that a wrong chain index or a different tree changes the bits."""
    rng = _rng(K)
    x = (rng.standard_normal(K) * np.exp2(rng.integers(-12, 12, K))).astype(np.float32)
    y = (rng.standard_normal(K) * np.exp2(rng.integers(-12, 12, K))).astype(np.float32)
    want = sdot32_exact(x, y)
    assert O.dot_f32(x, y).view(np.uint32) == want.view(np.uint32)


def test_sdot32_order_is_observable():
    """Guard for the test above: a plain left-to-right chain gives different bits on its inputs."""
    rng = _rng(64)
    x = (rng.standard_normal(64) * np.exp2(rng.integers(-12, 12, 64))).astype(np.float32)
    y = (rng.standard_normal(64) * np.exp2(rng.integers(-12, 12, 64))).astype(np.float32)
    serial = np.float32(0.0)
    for i in range(64):
        serial = fma32(x[i], y[i], serial)
    assert serial.view(np.uint32) != sdot32_exact(x, y).view(np.uint32)


@pytest.mark.skipif(not O.lib().trq_avx2_available(), reason="host has no AVX2/FMA/F16C")
def test_avx2_sdot32_matches_scalar():
    """Two independent restatements (scalar chains, and AVX2 intrinsics following cpu_gemv_amd64.s:190-227)."""
    import ctypes
    rng = _rng(5)
    for K in (32, 256, 4096, 14336):
        x = rng.standard_normal(K).astype(np.float32)
        y = rng.standard_normal(K).astype(np.float32)
        a = np.float32(O.lib().trq_avx2_sdot32(K, x.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p)))
        assert a.view(np.uint32) == O.dot_f32(x, y).view(np.uint32), K


@pytest.mark.parametrize("dt", DTS)
def test_quant_dot_equals_dequant_then_dot(dt):
    """TestQuantDotMatchesOpenedDot (cpu_quant_test.go:22-50): decoding in registers changes no bit."""
    rng = _rng(dt)
    K = 4 * 256
    w = O.small_scale_quant(dt, 11 + dt, K // BLOCK[dt][0])
    x = rng.standard_normal(K).astype(np.float32)
    assert O.quant_dot(dt, x, w).view(np.uint32) == O.dot_f32(x, O.dequant(dt, w)).view(np.uint32)


@pytest.mark.skipif(not O.lib().trq_avx2_available(), reason="host has no AVX2/FMA/F16C")
@pytest.mark.parametrize("dt", DTS)
def test_avx2_quant_dot_matches_scalar(dt):
    """sdotq8/q4/q4k/q6k restated from cpu_quant_amd64.s agree with the scalar restatement bit for bit,
    including the random (full fp16 range) blocks of the golden generator."""
    rng = _rng(10 + dt)
    for K, maker in ((4096, O.small_scale_quant), (512, O.random_quant)):
        w = maker(dt, 21 + dt, K // BLOCK[dt][0])
        x = rng.standard_normal(K).astype(np.float32)
        a, s = O.avx2_quant_dot(dt, x, w), O.quant_dot(dt, x, w)
        assert a.view(np.uint32) == s.view(np.uint32) or (np.isnan(a) and np.isnan(s))


@pytest.mark.parametrize("dt", DTS)
def test_quant_dot_close_to_float64(dt):
    """|got - sum x.deq(w)| <= 0.02 * sum |x.deq(w)| + 1e-6 (cpu_quant_q8_test.go:84)."""
    rng = _rng(30 + dt)
    K = 2048
    w = O.small_scale_quant(dt, 31, K // BLOCK[dt][0])
    x = rng.standard_normal(K).astype(np.float32)
    y = O.dequant(dt, w).astype(np.float64)
    want = float(np.dot(x.astype(np.float64), y))
    assert abs(float(O.quant_dot(dt, x, w)) - want) <= 0.02 * float(np.abs(x * y).sum()) + 1e-6


# ---------------------------------------------------------------- M>1 fp32 path (a11, a12)
def test_quant_gemm_single_row_is_gemv():
    rng = _rng(41)
    N, K = 7, 512
    w = O.small_scale_quant(Q4K, 42, N * K // 256)
    x = rng.standard_normal(K).astype(np.float32)
    c0 = rng.standard_normal(N).astype(np.float32)
    got = O.quant_gemm(Q4K, 1, N, K, x, w, c0)[0]
    rb = K // 256 * 144
    want = np.array([c0[n] + O.quant_dot(Q4K, x, w[n * rb:(n + 1) * rb]) for n in range(N)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quant_gemm_chunk_order_exactly():
    """M>1 (cpu_quant.go:47-83 with the panel micro-kernel): per output, each 256-deep K chunk is a fresh FMA
    chain in k order, chunks are added in order into part, then c += part. Restated with exact rationals."""
    rng = _rng(43)
    M, N, K = 2, 3, 768
    w = O.small_scale_quant(Q8, 44, N * K // 32)
    a = (rng.standard_normal((M, K)) * np.exp2(rng.integers(-6, 6, (M, K)))).astype(np.float32)
    c0 = rng.standard_normal(M * N).astype(np.float32)
    got = O.quant_gemm(Q8, M, N, K, a, w, c0).reshape(-1)
    deq = O.dequant(Q8, w).reshape(N, K)
    for m in range(M):
        for n in range(N):
            part = np.float32(0.0)
            for p0 in range(0, K, 256):
                chain = np.float32(0.0)
                for k in range(p0, p0 + 256):
                    chain = fma32(a[m, k], deq[n, k], chain)
                part = add32(part, chain)
            want = add32(c0[m * N + n], part)
            assert got[m * N + n].view(np.uint32) == want.view(np.uint32), (m, n)


@pytest.mark.parametrize("dt", DTS)
def test_quant_gemm_empty_sum(dt):
    """K == 0 leaves c unchanged (TestQuantMatMulEmptySum, cpu_quant_test.go:262)."""
    c0 = np.arange(6, dtype=np.float32)
    got = O.quant_gemm(dt, 2, 3, 0, np.zeros(0, np.float32), np.zeros(0, np.uint8), c0)
    assert np.array_equal(got.reshape(-1), c0)


# ---------------------------------------------------------------- activation quantizer (a13)
def test_quantize_q8_k_edge_blocks():
    g = {c["name"]: c for c in GOLD["quantize_q8_k_edges"]["cases"]}
    tiny = np.array([0x00400000], np.uint32).view(np.float32)[0]
    fills = {
        "zero": np.zeros(256, np.float32),
        "saturate": np.where(np.arange(256) % 2 == 1, -3.0, 3.0).astype(np.float32),
        "one_large": np.full(256, 1e-3, np.float32),
        "tiny": np.zeros(256, np.float32),
    }
    fills["one_large"][5] = 1000
    fills["tiny"][0], fills["tiny"][1], fills["tiny"][2] = tiny, -tiny / 2, tiny / 4
    for name, x in fills.items():
        q, d, bs = O.quantize_q8(x, 256)
        c = g[name]
        assert d[0] == np.float32(c["d_num"]) / np.float32(c["d_den"]), name
        want = np.zeros(256, np.int8)
        if name == "saturate":
            want = np.where(np.arange(256) % 2 == 1, -127, 127).astype(np.int8)
        for k, v in c.get("codes", {}).items():
            want[int(k)] = v
        assert np.array_equal(q, want), name
        assert np.array_equal(bs, q.reshape(16, 16).astype(np.int16).sum(axis=1).astype(np.int16)), name


def test_quantize_q8_block_edges_two_blocks():
    """Each 32-block's scale comes from its own elements; the tie 0.5*127 = 63.5 rounds to even 64."""
    t = GOLD["quantize_q8_block_edges"]["two_block"]
    x = np.full(64, 0.5, np.float32)
    x[32:] = 1000
    x[0] = 1
    q, d, _ = O.quantize_q8(x, 32)
    assert d[0] == np.float32(t["d0_num"]) / np.float32(t["d0_den"])
    assert d[1] == np.float32(t["d1_num"]) / np.float32(t["d1_den"])
    assert (q[0], q[1], q[32]) == (t["q0"], t["q1"], t["q32"])


@pytest.mark.parametrize("blk", [32, 256])
def test_quantize_q8_random_matches_float32_rule(blk):
    """amax; id = fl(127/amax); q = clamp(rne(fl(x*id)), +-127); d = fl(amax/127) -- numpy float32 ops are
    individually rounded, so this is the rule of cpu_quant_q8.go:39-68 evaluated independently."""
    rng = _rng(blk)
    x = (rng.standard_normal(4 * blk) * np.exp2(rng.integers(-20, 20, 4 * blk))).astype(np.float32)
    q, d, bs = O.quantize_q8(x, blk)
    xb = x.reshape(-1, blk)
    amax = np.abs(xb).max(axis=1)
    idv = (np.float32(127.0) / amax).astype(np.float32)
    want = np.clip(np.rint((xb * idv[:, None]).astype(np.float32)), -127, 127).astype(np.int8).reshape(-1)
    assert np.array_equal(q, want)
    assert np.array_equal(d, (amax / np.float32(127.0)).astype(np.float32))


# ---------------------------------------------------------------- act-quant block kernels (a15-a18)
def _unit_scales(dt, raw, mode):
    """Copy of raw blocks with d = 1 (mode 'd') or, for q4_k, d = 0 and dmin = 1 (mode 'm')."""
    r = raw.copy().reshape(-1, BLOCK[dt][1])
    one, zero = (0x00, 0x3C), (0x00, 0x00)
    if dt == Q4:
        r[:, 0], r[:, 1] = one
    elif dt == Q4K:
        (r[:, 0], r[:, 1]), (r[:, 2], r[:, 3]) = (one, zero) if mode == "d" else (zero, one)
    elif dt == Q6K:
        r[:, 208], r[:, 209] = one
    return r.reshape(-1)


@pytest.mark.parametrize("dt", [Q4, Q4K, Q6K])
def test_block_isums_brute_force(dt):
    """The integer block sums equal int64 brute force over the codes. The codes and scales are read back from
    the golden-pinned dequantization of the same bytes with d = 1 (and dmin = 1 for the q4_k min term)."""
    rng = _rng(50 + dt)
    be = BLOCK[dt][0]
    nb = 8 if be == 32 else 4
    K = nb * be
    raw = O.random_quant(dt, 60 + dt, nb)
    x = rng.standard_normal(K).astype(np.float32)
    q, _, bs = O.quantize_q8(x, be)
    isum, msum = O.block_isums(dt, raw, q, bs)
    qq = q.astype(np.int64).reshape(nb, be)
    yd = O.dequant(dt, _unit_scales(dt, raw, "d")).astype(np.float64).reshape(nb, be)
    assert np.all(yd == np.round(yd))
    if dt == Q4:
        assert np.array_equal(isum, (yd.astype(np.int64) * qq).sum(axis=1))
    elif dt == Q4K:
        # d = 1, dmin = 0 -> y = sc_j * q ; d = 0, dmin = 1 -> y = -m_j
        assert np.array_equal(isum, (yd.astype(np.int64) * qq).sum(axis=1))
        ym = O.dequant(dt, _unit_scales(dt, raw, "m")).astype(np.int64).reshape(nb, be)
        assert np.array_equal(msum, (-ym * qq).sum(axis=1))
    else:
        # d = 1 -> y = sc * (q6 - 32); the epilogue uses isum - 32 msum
        assert np.array_equal(isum.astype(np.int64) - 32 * msum.astype(np.int64), (yd.astype(np.int64) * qq).sum(axis=1))


@pytest.mark.parametrize("dt", [Q4, Q4K, Q6K])
def test_quant_gemm_act_epilogue(dt):
    """Output = blocks in order, each with the float32 epilogue of cpu_quant_q8.go (no FMA), over the
    brute-force-checked integer sums; rows are independent (x4/x8 == x1)."""
    rng = _rng(70 + dt)
    be = BLOCK[dt][0]
    M, N, K = 3, 4, 2 * 256
    nb = K // be
    w = O.small_scale_quant(dt, 71, N * nb)
    a = rng.standard_normal((M, K)).astype(np.float32)
    c0 = rng.standard_normal(M * N).astype(np.float32)
    got = O.quant_gemm_act(dt, M, N, K, a, w, c0)
    f32 = np.float32
    for m in range(M):
        q, d8, bs = O.quantize_q8(a[m], be)
        for n in range(N):
            row = w[n * nb * BLOCK[dt][1]:(n + 1) * nb * BLOCK[dt][1]]
            isum, msum = O.block_isums(dt, row, q, bs)
            acc = f32(0.0)
            blocks = row.reshape(nb, BLOCK[dt][1])
            for b in range(nb):
                if dt == Q4:
                    dw = blocks[b, :2].view(np.float16).astype(f32)[0]
                    acc = f32(acc + f32(f32(dw * d8[b]) * f32(isum[b])))
                elif dt == Q4K:
                    dw = blocks[b, :2].view(np.float16).astype(f32)[0]
                    dm = blocks[b, 2:4].view(np.float16).astype(f32)[0]
                    t = f32(f32(dw * f32(isum[b])) - f32(dm * f32(msum[b])))
                    acc = f32(acc + f32(t * d8[b]))
                else:
                    dw = blocks[b, 208:210].view(np.float16).astype(f32)[0]
                    t = f32(dw * f32(int(isum[b]) - 32 * int(msum[b])))
                    acc = f32(acc + f32(t * d8[b]))
            want = f32(c0[m * N + n] + acc)
            assert got[m, n].view(np.uint32) == want.view(np.uint32), (m, n)
        one = O.quant_gemm_act(dt, 1, N, K, a[m], w, c0[m * N:(m + 1) * N])
        assert np.array_equal(one.view(np.uint32), got[m:m + 1].view(np.uint32))


@pytest.mark.skipif(not O.lib().trq_avx2_available(), reason="host has no AVX2/FMA/F16C")
@pytest.mark.parametrize("dt", [Q4, Q4K, Q6K])
def test_avx2_act_quant_matches_scalar(dt):
    import ctypes
    rng = _rng(80 + dt)
    M, N, K = 5, 6, 4096
    w = O.small_scale_quant(dt, 81, N * K // BLOCK[dt][0])
    a = rng.standard_normal((M, K)).astype(np.float32)
    c = np.zeros(M * N, np.float32)
    P = ctypes.c_void_p
    O.lib().trq_avx2_quant_gemm_act(dt, M, N, K, a.ctypes.data_as(P), w.ctypes.data_as(P), c.ctypes.data_as(P), 2)
    assert np.array_equal(c.view(np.uint32), O.quant_gemm_act(dt, M, N, K, a, w).reshape(-1).view(np.uint32))


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_act_quant_non_finite_row_takes_float_path(bad):
    """TestQ8PathKeepsNonFinite (cpu_quant_q8_test.go:471): the row with NaN/Inf equals the fp32 GEMV of that
    row alone; the other rows are the quantized results."""
    rng = _rng(90)
    M, N, K = 3, 5, 512
    w = O.small_scale_quant(Q4K, 91, N * K // 256)
    a = rng.standard_normal((M, K)).astype(np.float32)
    a[1, 17] = bad
    got = O.quant_gemm_act(Q4K, M, N, K, a, w)
    same = lambda u, v: np.array_equal(np.isnan(u), np.isnan(v)) and np.array_equal(
        u[~np.isnan(u)].view(np.uint32), v[~np.isnan(v)].view(np.uint32))
    assert same(got[1], O.quant_gemm(Q4K, 1, N, K, a[1], w)[0])
    for m in (0, 2):
        assert same(got[m], O.quant_gemm_act(Q4K, 1, N, K, a[m], w)[0])


# ---------------------------------------------------------------- embedding (next row 3)
@pytest.mark.parametrize("dt", DTS)
def test_embedding_is_dequantized_rows(dt):
    D = 512
    raw = O.random_quant(dt, 95, 5 * D // BLOCK[dt][0])
    rows = O.dequant(dt, raw).reshape(5, D)
    idx = [4, 0, 4, 2]
    got = O.embedding(dt, raw, D, idx)
    assert np.array_equal(np.isnan(got), np.isnan(rows[idx]))
    fin = ~np.isnan(got)
    assert np.array_equal(got[fin].view(np.uint32), rows[idx][fin].view(np.uint32))


# ---------------------------------------------------------------- SwiGLU epilogue (exp, silu)
def _ulps(got, want):
    """|got - want| in units of want's float32 spacing (cpu_math_test.go:9-23 ulpDiff)."""
    got = np.asarray(got, np.float64)
    want32 = np.asarray(want, np.float32)
    sp = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got - want32.astype(np.float64)) / sp


def test_exp_vec_within_two_ulp():
    """expVec within 2 ulp of float32(math.Exp) over the reference's own sample (cpu_math_test.go:89-120):
    uniform [-115, 105), its edge list and small integers."""
    rng = np.random.default_rng(43)
    xs = (rng.random(200000) * 220 - 115).astype(np.float32)
    edges = np.array([0, -0.0, 88.7, 88.72283, 88.7229, 89, 1000, -87.33654, -87.34, -95, -100, -103.9, -103.97,
                      -104, -150, 1e-8, -1e-8] + [k - 4 for k in range(9)], np.float32)
    xs = np.concatenate([xs, edges])
    got = O.exp_vec(xs)
    with np.errstate(over="ignore"):
        want = np.exp(xs.astype(np.float64)).astype(np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[~fin], want[~fin])
    assert float(np.max(_ulps(got[fin], want[fin]))) <= 2


def test_exp_vec_special_values():
    """cpu_math_test.go:50-54: e^89 = +Inf, e^-200 = 0, e^-Inf = 0; NaN passes; e^0 = 1 exactly."""
    got = O.exp_vec(np.array([89, -200, -np.inf, np.inf, np.nan, 0, -0.0], np.float32))
    assert got[0] == np.inf and got[1] == 0 and got[2] == 0 and got[3] == np.inf
    assert np.isnan(got[4]) and got[5] == 1 and got[6] == 1


def test_silu_within_three_ulp():
    """siluForward within 3 ulp of x / (1 + e^-x) in float64 (elementwise_wide_test.go:35-40, 69-70) on a fine
    grid over [-20, 20] and N(0, 5) samples."""
    rng = np.random.default_rng(7)
    xs = np.concatenate([np.arange(-20, 20, 0.001, dtype=np.float32), (rng.standard_normal(20000) * 5).astype(np.float32)])
    got = O.silu(xs)
    x64 = xs.astype(np.float64)
    want = (x64 / (1 + np.exp(-x64))).astype(np.float32)
    assert float(np.max(_ulps(got, want))) <= 3


def test_silu_special_values():
    """silu(-Inf) = 0 and silu(+Inf) = +Inf (elementwise_wide_test.go:158-159); the sign of -0 stays; NaN stays;
    large negative x gives +0 once sigma underflows (cpu_elementwise_wide.go:109-111)."""
    got = O.silu(np.array([-np.inf, np.inf, -0.0, np.nan, -200, 0], np.float32))
    assert got[0] == 0 and not np.signbit(got[0])
    assert got[1] == np.inf
    assert got[2] == 0 and np.signbit(got[2])
    assert np.isnan(got[3])
    assert got[4] == 0 and not np.signbit(got[4])
    assert got[5] == 0 and not np.signbit(got[5])


def test_swiglu_gate_is_first_half():
    """The merged gate_up output is [G | U] per row (layers.tr:240-262 .split(2)): gate values enter silu."""
    M, I = 3, 5
    g = np.arange(M * I, dtype=np.float32).reshape(M, I) / 7 - 1
    u = np.full((M, I), 2.0, np.float32)
    out = O.swiglu(np.concatenate([g, u], axis=1), M, I)
    assert np.array_equal(out, (O.silu(g).reshape(M, I) * np.float32(2)).astype(np.float32))


# ---- 16-bit activations and outputs: the reference's rounding and widening (tensor/cpu_dtype.go:73-145)

def _f32(b):
    return np.array([b], np.uint32).view(np.float32)[0]


BF16_EDGES = [  # tensor/dtype_test.go:17-34
    (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3F80), (-2.0, 0xC000),
    (1 + 1.0 / 256, 0x3F80), (1 + 3.0 / 256, 0x3F82), (1 + 1.0 / 256 + 1.0 / (1 << 20), 0x3F81),
    (_f32(0x7F7FFFFF), 0x7F80), (-_f32(0x7F7FFFFF), 0xFF80), (_f32(0x7F7F0000), 0x7F7F),
    (np.inf, 0x7F80), (-np.inf, 0xFF80), (_f32(0x00010000), 0x0001), (_f32(0x00008000), 0x0000),
    (_f32(0x00018000), 0x0002)]
F16_EDGES = [  # tensor/dtype_test.go:52-75
    (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (65519.0, 0x7BFF),
    (65520.0, 0x7C00), (1e6, 0x7C00), (-1e6, 0xFC00), (1 + 1.0 / 2048, 0x3C00), (1 + 3.0 / 2048, 0x3C02),
    (6.103515625e-05, 0x0400), (5.960464477539063e-08, 0x0001), (2.9802322387695312e-08, 0x0000),
    (2.9802322387695312e-08 * 1.0001, 0x0001), (4.470348358154297e-08, 0x0001), (8.940696716308594e-08, 0x0002),
    (6.097555160522461e-05, 0x03FF), (6.1005353927612305e-05, 0x0400), (1e-10, 0x0000), (-1e-10, 0x8000),
    (np.inf, 0x7C00), (-np.inf, 0xFC00)]


@pytest.mark.parametrize("t,cases", [(2, BF16_EDGES), (1, F16_EDGES)])
def test_round16_reference_edges(t, cases):
    """The reference's known answers for float32 -> bfloat16 / float16 (ties to even, overflow, subnormals)."""
    x = np.array([c[0] for c in cases], np.float32)
    want = np.array([c[1] for c in cases], np.uint16)
    assert np.array_equal(O.round16(t, x), want)


@pytest.mark.parametrize("t", [1, 2])
def test_round16_nan_and_round_trip(t):
    """NaN stays NaN (bfloat16: quieted by 0x0040, tensor/dtype_test.go:42-47); every non-NaN 16-bit pattern widens
    exactly and rounds back to itself (tensor/dtype_test.go:91-100)."""
    nans = np.array([0x7FC00000, 0x7F800001, 0xFFC00000, 0x7F80FFFF], np.uint32).view(np.float32)
    h = O.round16(t, nans)
    assert np.all(np.isnan(O.widen16(t, h)))
    if t == 2:
        assert np.all(h & 0x0040)
    allbits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    wide = O.widen16(t, allbits)
    keep = ~np.isnan(wide)
    assert np.array_equal(O.round16(t, wide[keep]), allbits[keep])
    if t == 1:  # the f16 widening agrees with numpy's for every non-NaN pattern
        assert np.array_equal(wide[keep].view(np.uint32), allbits[keep].view(np.float16).astype(np.float32).view(np.uint32))


def test_round16_nearest_even_on_random_floats():
    """float16: numpy's IEEE conversion (round to nearest even) on finite values of every magnitude. bfloat16: the
    result is the nearest of its neighbours, ties to the even pattern."""
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, size=200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        assert np.array_equal(O.round16(1, x), x.astype(np.float16).view(np.uint16))
    h = O.round16(2, x).astype(np.int64)
    xd = x.astype(np.float64)
    fin = np.abs(xd) < float(_f32(0x7F7F8000))  # below the bfloat16 overflow threshold
    h, xd = h[fin], xd[fin]
    inner = ((h & 0x7FFF) > 0) & ((h & 0x7FFF) < 0x7F7F)  # both neighbours are finite patterns of the same sign
    h, xd = h[inner], xd[inner]
    mag = h & 0x7FFF
    sign = h & 0x8000
    w = lambda m: O.widen16(2, (sign | m).astype(np.uint16)).astype(np.float64)
    d0 = np.abs(xd - w(mag))
    assert np.all(d0 <= np.abs(xd - w(mag + 1))) and np.all(d0 <= np.abs(xd - w(mag - 1)))
    tie = (d0 == np.abs(xd - w(mag + 1))) | (d0 == np.abs(xd - w(mag - 1)))
    assert np.all((mag[tie & (d0 > 0)] & 1) == 0)
