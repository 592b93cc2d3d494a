"""ctypes view of the CPU oracle (oracle/liboracle.so) for the tests: expected results only."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATH = os.path.join(ROOT, "oracle", "liboracle.so")
P = ctypes.c_void_p
SZ = ctypes.c_size_t

_L = None


def lib():
    global _L
    if _L is None:
        if not os.path.exists(PATH):
            raise ImportError("oracle not built: %s" % PATH)
        L = ctypes.CDLL(PATH)
        L.trq_f16_to_f32.restype = ctypes.c_float
        L.trq_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.trq_dot_f32.restype = ctypes.c_float
        L.trq_dot_f32.argtypes = [P, P, SZ]
        L.trq_quant_dot.restype = ctypes.c_float
        L.trq_quant_dot.argtypes = [ctypes.c_int, P, P, SZ]
        L.trq_avx2_quant_dot.restype = ctypes.c_float
        L.trq_avx2_quant_dot.argtypes = [ctypes.c_int, P, P, SZ]
        L.trq_avx2_sdot32.restype = ctypes.c_float
        L.trq_avx2_sdot32.argtypes = [SZ, P, P]
        L.trq_fnv1a64_f32.restype = ctypes.c_uint64
        L.trq_fnv1a64_f32.argtypes = [P, SZ]
        L.trq_check_quant_scales.restype = ctypes.c_long
        L.trq_check_quant_scales.argtypes = [ctypes.c_int, P, SZ]
        for name in ("trq_dot_q4q8",):
            getattr(L, name).restype = ctypes.c_float
            getattr(L, name).argtypes = [SZ, P, P, P]
        for name in ("trq_dot_q4kq8", "trq_dot_q6kq8"):
            getattr(L, name).restype = ctypes.c_float
            getattr(L, name).argtypes = [SZ, P, P, P, P]
        L.trq_random_quant.argtypes = [ctypes.c_int, ctypes.c_uint32, SZ, P]
        L.trq_dequant.argtypes = [ctypes.c_int, P, SZ, P]
        L.trq_quant_zero_raw.argtypes = [ctypes.c_int, SZ, P]
        L.trq_quant_gemm.argtypes = [ctypes.c_int, SZ, SZ, SZ, P, P, P, ctypes.c_int]
        L.trq_quant_gemm_act.argtypes = [ctypes.c_int, SZ, SZ, SZ, P, P, P, ctypes.c_int]
        L.trq_avx2_quant_gemv.argtypes = [ctypes.c_int, SZ, SZ, P, P, P, ctypes.c_int]
        L.trq_avx2_quant_gemm_act.argtypes = [ctypes.c_int, SZ, SZ, SZ, P, P, P, ctypes.c_int]
        L.trq_quantize_q8.argtypes = [P, SZ, ctypes.c_int, P, P, P]
        L.trq_block_isums.argtypes = [ctypes.c_int, SZ, P, P, P, P, P]
        L.trq_quant_embedding.argtypes = [ctypes.c_int, P, SZ, P, SZ, P]
        for name in ("trq_exp_vec", "trq_silu"):
            getattr(L, name).restype = ctypes.c_float
            getattr(L, name).argtypes = [ctypes.c_float]
        L.trq_swiglu.argtypes = [P, SZ, SZ, P]
        _L = L
    return _L


def _p(a):
    return a.ctypes.data_as(P)


BLOCK = {1: (32, 34), 2: (32, 18), 3: (256, 144), 4: (256, 210)}
THREADS = min(8, os.cpu_count() or 1)


def random_quant(dt, seed, blocks):
    out = np.zeros(blocks * BLOCK[dt][1], np.uint8)
    lib().trq_random_quant(dt, seed & 0xFFFFFFFF, blocks, _p(out))
    return out


def small_scale_quant(dt, seed, blocks):
    """cpu_quant_test.go:71-86: random blocks with fp16 scales forced to moderate magnitudes."""
    raw = random_quant(dt, seed, blocks).reshape(blocks, BLOCK[dt][1])
    if dt in (1, 2):
        raw[:, 1] = 0x1C | (raw[:, 1] & 0x83)
    elif dt == 3:
        raw[:, 1] = 0x1C | (raw[:, 1] & 0x83)
        raw[:, 3] = 0x1C | (raw[:, 3] & 0x83)
    else:
        raw[:, 209] = 0x1C | (raw[:, 209] & 0x83)
    return raw.reshape(-1)


def dequant(dt, raw):
    nb = raw.size // BLOCK[dt][1]
    y = np.zeros(nb * BLOCK[dt][0], np.float32)
    lib().trq_dequant(dt, _p(raw), nb, _p(y))
    return y


def fnv(y):
    y = np.ascontiguousarray(y, np.float32)
    return lib().trq_fnv1a64_f32(_p(y), y.size)


def quant_dot(dt, x, w):
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().trq_quant_dot(dt, _p(x), _p(w), x.size))


def avx2_quant_dot(dt, x, w):
    x = np.ascontiguousarray(x, np.float32)
    return np.float32(lib().trq_avx2_quant_dot(dt, _p(x), _p(w), x.size))


def dot_f32(x, y):
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    return np.float32(lib().trq_dot_f32(_p(x), _p(y), x.size))


def quant_gemm(dt, M, N, K, a, w, c=None):
    a = np.ascontiguousarray(a, np.float32)
    c = np.zeros(M * N, np.float32) if c is None else np.ascontiguousarray(c, np.float32).copy()
    lib().trq_quant_gemm(dt, M, N, K, _p(a), _p(w), _p(c), THREADS)
    return c.reshape(M, N)


def quant_gemm_act(dt, M, N, K, a, w, c=None):
    a = np.ascontiguousarray(a, np.float32)
    c = np.zeros(M * N, np.float32) if c is None else np.ascontiguousarray(c, np.float32).copy()
    lib().trq_quant_gemm_act(dt, M, N, K, _p(a), _p(w), _p(c), THREADS)
    return c.reshape(M, N)


def quantize_q8(x, blk):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    K = x.size
    q = np.zeros(K, np.int8)
    d = np.zeros(K // blk, np.float32)
    bs = np.zeros(K // 16, np.int16)
    lib().trq_quantize_q8(_p(x), K, blk, _p(q), _p(d), _p(bs))
    return q, d, bs


def block_isums(dt, w_row, q, bs):
    nb = q.size // BLOCK[dt][0]
    isum = np.zeros(nb, np.int32)
    msum = np.zeros(nb, np.int32)
    lib().trq_block_isums(dt, nb, _p(w_row), _p(q), _p(bs), _p(isum), _p(msum))
    return isum, msum


def round16(t, x):
    """float32 array -> uint16 patterns of type t (1 = f16, 2 = bf16), cpu_dtype.go:73-123."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(x.size, np.uint16)
    lib().trq_round16(t, _p(x), _p(out), SZ(x.size))
    return out


def widen16(t, h):
    """uint16 patterns of type t -> float32 (exact), cpu_dtype.go:83, :125-145."""
    h = np.ascontiguousarray(h, np.uint16).reshape(-1)
    out = np.zeros(h.size, np.float32)
    lib().trq_widen16(t, _p(h), _p(out), SZ(h.size))
    return out


def quant_zero_raw(dt, n):
    out = np.zeros(n // BLOCK[dt][0] * BLOCK[dt][1], np.uint8)
    lib().trq_quant_zero_raw(dt, n, _p(out))
    return out


def check_quant_scales(dt, raw):
    return lib().trq_check_quant_scales(dt, _p(raw), raw.size)


def embedding(dt, raw, D, idx):
    idx = np.ascontiguousarray(idx, np.int64)
    out = np.zeros(idx.size * D, np.float32)
    lib().trq_quant_embedding(dt, _p(raw), D, _p(idx), idx.size, _p(out))
    return out.reshape(idx.size, D)


def exp_vec(x):
    """e^x elementwise as the reference's AVX2 expVec (scalar loop over trq_exp_vec)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    f = lib().trq_exp_vec
    return np.array([f(float(v)) for v in x], np.float32)


def silu(x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    f = lib().trq_silu
    return np.array([f(float(v)) for v in x], np.float32)


def swiglu(gu, M, I):
    gu = np.ascontiguousarray(gu, np.float32).reshape(-1)
    out = np.zeros(M * I, np.float32)
    lib().trq_swiglu(_p(gu), M, I, _p(out))
    return out.reshape(M, I)
