"""Synthetic inputs and GGUF block encoders (host, numpy).

Seeded generator: splitmix64 -> two uniforms -> Box-Muller in float64 -> float32. The same seed gives
the same bytes on every machine, so the CPU baseline and the GPU see identical inputs.

Encoders:
  q8   llama.cpp Q8_0 (the reference's "q8", docs/spec/15_tensorler.md:670-671): d = amax/127 in float32,
       code = round-half-away(x * (1/d)), d stored as fp16 (round to nearest even).
  q4   llama.cpp Q4_0 (spec :672): d = (signed element of largest |x|)/-8, code = min(15, trunc(x/d + 8.5)).
  q4_k, q6_k: TR has no encoder for these (spec :664, read-only formats). This module's own
       round-to-nearest encoders fill the same block layouts (tensor/quant.go:23-47); they only produce
       test weights and are not part of the matmul being checked.
"""
import numpy as np

from ._lib import Q8, Q4, Q4K, Q6K

_M64 = (1 << 64) - 1


def _splitmix64(n, seed):
    """n consecutive splitmix64 outputs for state seed."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & _M64) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def normal(n, seed, std=1.0):
    """n float32 samples of N(0, std^2)."""
    m = (n + 1) // 2
    u = _splitmix64(2 * m, seed)
    u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)  # (0, 1]
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:n] * std).astype(np.float32)


def weights_f32(N, K, seed, std=0.02, outliers=0.0):
    """[N, K] float32 weights ~ N(0, std^2); a seeded fraction `outliers` of entries is scaled x10."""
    w = normal(N * K, seed, std).reshape(N, K)
    if outliers > 0:
        u = _splitmix64(N * K, seed ^ 0x5EED0F)
        pick = (u >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0) < outliers
        w.reshape(-1)[pick] *= np.float32(10.0)
    return w


def _f16_bits(v):
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint16)


def _round_half_away(v):
    v = np.asarray(v, dtype=np.float64)  # exact for float32 inputs
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def encode_q8_0(x):
    """[N, K] float32 -> Q8_0 blocks (34 B per 32 elements), llama.cpp quantize_row_q8_0_ref."""
    N, K = x.shape
    b = x.reshape(N, K // 32, 32).astype(np.float32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    q = _round_half_away((b * idv[..., None]).astype(np.float32)).astype(np.int8)
    out = np.empty((N, K // 32, 34), dtype=np.uint8)
    out[..., 0:2] = _f16_bits(d).reshape(N, K // 32, 1).view(np.uint8).reshape(N, K // 32, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(-1)


def encode_q4_0(x):
    """[N, K] float32 -> Q4_0 blocks (18 B per 32 elements), llama.cpp quantize_row_q4_0_ref."""
    N, K = x.shape
    b = x.reshape(N, K // 32, 32).astype(np.float32)
    # signed element of the largest magnitude; the first one wins a tie (strictly greater test)
    idx = np.argmax(np.abs(b), axis=2)
    mx = np.take_along_axis(b, idx[..., None], axis=2)[..., 0]
    mx = np.where(np.abs(mx) > 0, mx, np.float32(0.0)).astype(np.float32)
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = (b * idv[..., None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(15, np.trunc(v.astype(np.float32)).astype(np.int32)).astype(np.uint8)
    out = np.empty((N, K // 32, 18), dtype=np.uint8)
    out[..., 0:2] = _f16_bits(d).reshape(N, K // 32, 1).view(np.uint8).reshape(N, K // 32, 2)
    out[..., 2:] = (q[..., :16] | (q[..., 16:] << 4)).astype(np.uint8)
    return out.reshape(-1)


def _f16(v):
    return np.asarray(v, dtype=np.float32).astype(np.float16).astype(np.float32)


def encode_q4_k(x):
    """[N, K] float32 -> Q4_K blocks (144 B per 256): per 32-element sub-block an asymmetric
    round-to-nearest fit with 6-bit scale/min, block d/dmin in fp16."""
    N, K = x.shape
    nb = K // 256
    b = x.reshape(N, nb, 8, 32).astype(np.float32)
    mn = np.minimum(b.min(axis=3), 0.0).astype(np.float32)
    mx = b.max(axis=3).astype(np.float32)
    scale = ((mx - mn) / 15.0).astype(np.float32)
    mins = (-mn).astype(np.float32)
    d = _f16(scale.max(axis=2) / 63.0)
    dmin = _f16(mins.max(axis=2) / 63.0)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[..., None] > 0, np.rint(scale / d[..., None]), 0)
        m = np.where(dmin[..., None] > 0, np.rint(mins / dmin[..., None]), 0)
    sc = np.clip(sc, 0, 63).astype(np.uint8)
    m = np.clip(m, 0, 63).astype(np.uint8)
    d1 = (d[..., None] * sc).astype(np.float32)
    m1 = (dmin[..., None] * m).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(d1[..., None] > 0, np.rint((b + m1[..., None]) / d1[..., None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint8)  # [N, nb, 8, 32]
    out = np.zeros((N, nb, 144), dtype=np.uint8)
    out[..., 0:2] = _f16_bits(d).reshape(N, nb, 1).view(np.uint8).reshape(N, nb, 2)
    out[..., 2:4] = _f16_bits(dmin).reshape(N, nb, 1).view(np.uint8).reshape(N, nb, 2)
    s = np.zeros((N, nb, 12), dtype=np.uint8)
    # inverse of q4kScale (tensor/quant.go:158-163)
    s[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    s[..., 4:8] = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    s[..., 8:12] = (sc[..., 4:8] & 0xF) | ((m[..., 4:8] & 0xF) << 4)
    out[..., 4:16] = s
    qs = q[:, :, 0::2, :] | (q[:, :, 1::2, :] << 4)  # [N, nb, 4, 32]: low = sub-block 2g, high = 2g+1
    out[..., 16:] = qs.reshape(N, nb, 128)
    return out.reshape(-1)


def encode_q6_k(x):
    """[N, K] float32 -> Q6_K blocks (210 B per 256): per 16-element sub-block a symmetric
    round-to-nearest fit with int8 scale, block d in fp16."""
    N, K = x.shape
    nb = K // 256
    b = x.reshape(N, nb, 16, 16).astype(np.float32)
    s = (np.abs(b).max(axis=3) / 31.0).astype(np.float32)
    d = _f16(s.max(axis=2) / 127.0)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[..., None] > 0, np.rint(s / d[..., None]), 0)
    sc = np.clip(sc, -128, 127).astype(np.int8)
    ds = (d[..., None] * sc.astype(np.float32)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(ds[..., None] != 0, np.rint(b / ds[..., None]), 0)
    code = (np.clip(q, -32, 31) + 32).astype(np.uint8).reshape(N, nb, 2, 4, 32)  # [half, k, l]
    ql = np.zeros((N, nb, 2, 64), dtype=np.uint8)
    qh = np.zeros((N, nb, 2, 32), dtype=np.uint8)
    ql[..., 0:32] = (code[:, :, :, 0] & 0xF) | ((code[:, :, :, 2] & 0xF) << 4)
    ql[..., 32:64] = (code[:, :, :, 1] & 0xF) | ((code[:, :, :, 3] & 0xF) << 4)
    qh[...] = (code[:, :, :, 0] >> 4) | ((code[:, :, :, 1] >> 4) << 2) | ((code[:, :, :, 2] >> 4) << 4) | ((code[:, :, :, 3] >> 4) << 6)
    out = np.zeros((N, nb, 210), dtype=np.uint8)
    out[..., 0:128] = ql.reshape(N, nb, 128)
    out[..., 128:192] = qh.reshape(N, nb, 64)
    out[..., 192:208] = sc.view(np.uint8)
    out[..., 208:210] = _f16_bits(d).reshape(N, nb, 1).view(np.uint8).reshape(N, nb, 2)
    return out.reshape(-1)


ENCODERS = {Q8: encode_q8_0, Q4: encode_q4_0, Q4K: encode_q4_k, Q6K: encode_q6_k}


def quant_weights(dt, N, K, seed, std=0.02, outliers=0.0, chunk_rows=128):
    """Seeded fp32 weights encoded to dtype dt, row chunk by row chunk (bounded memory)."""
    parts = []
    for r0 in range(0, N, chunk_rows):
        n = min(chunk_rows, N - r0)
        w = weights_f32(n, K, seed * 1000003 + r0, std, outliers)
        parts.append(ENCODERS[dt](w))
    return np.concatenate(parts) if parts else np.zeros(0, np.uint8)


def activations(M, K, seed):
    return normal(M * K, seed).reshape(M, K)


def random_blocks(dt, N, K, seed):
    """Blocks of uniformly random codes with moderate fp16 scales (d ~ 2^-7, q4_k dmin ~ 2^-8, q6_k signed
    scales kept): well-formed inputs for throughput runs over many large tensors, where encoding real weights
    would dominate the run time. Values are not meant to look like trained weights."""
    bb = {Q8: 34, Q4: 18, Q4K: 144, Q6K: 210}[dt]
    be = 32 if dt in (Q8, Q4) else 256
    nb = N * (K // be)
    rng = np.random.default_rng(seed)
    # at most 2^16 distinct random blocks, repeated: generating hundreds of MB of random bytes costs seconds
    uniq = min(nb, 1 << 16)
    base = np.frombuffer(rng.bytes(uniq * bb), dtype=np.uint8).reshape(uniq, bb)
    raw = np.resize(base, (nb, bb))
    d = _f16_bits(np.full(1, 2.0 ** -7, np.float32)).view(np.uint8)
    if dt in (Q8, Q4):
        raw[:, 0:2] = d
    elif dt == Q4K:
        raw[:, 0:2] = d
        raw[:, 2:4] = _f16_bits(np.full(1, 2.0 ** -8, np.float32)).view(np.uint8)
    else:
        raw[:, 208:210] = d
    return raw.reshape(-1)
