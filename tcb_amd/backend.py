"""Host-side mirror of TR's quantized-matmul operator interface over libtrhip.

Names and argument meaning follow the reference's Backend slice for this path
(internal/compute/tensor/device.go:378-512, matmul.go:59-61, quant.go:62-105, typed.go:22-30):

  QuantBackend.FromQuantized(dt, raw, N, K)      tensor/quant.go:62 (+ gpu FromRaw, gpu/typed.go:24-35)
  QuantBackend.Gemm(M, N, K, a, w, c)            Backend.Gemm, device.go:478 (c +=)
  QuantBackend.GemmSet(M, N, K, a, w, c)         GemmSetter.GemmSet, device_registry.go:193-195 (c =)
  QuantBackend.GemmActQuant(M, N, K, a, w, c)    ActQuantGemmer.GemmActQuant, matmul.go:59-61
  QuantBackend.OpenQuant(out, w, offset, n)      QuantOpener.OpenQuant, quant.go:103-105
  QuantBackend.Embedding(out, w, idx)            Backend.Embedding, device.go:482
  QuantBackend.NewQuantStorage(dt, N, K)        newQuantStorage / QuantZeroRaw, quant.go:408-427
  QuantWeight.ToRaw(row0, rows)                  RawBackend.ToRaw, typed.go:27
  CheckQuantScales(dt, raw)                      tensor/quant.go:108-128

Errors surface as TrhipError carrying the library's status code and detail text, the analogue of
the reference's coded panics (messages.New(H...)).
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import P, Q8, Q4, Q4K, Q6K, MODE_EXACT, MODE_FAST  # noqa: F401

BLOCK = {Q8: (32, 34), Q4: (32, 18), Q4K: (256, 144), Q6K: (256, 210)}  # tensor/quant.go:23-47
NAMES = {Q8: "q8", Q4: "q4", Q4K: "q4_k", Q6K: "q6_k"}
BY_NAME = {v: k for k, v in NAMES.items()}


class TrhipError(RuntimeError):
    def __init__(self, code, detail):
        self.code = code
        self.detail = detail
        name = _lib.lib().trhip_strerror(code).decode()
        super().__init__("trhip error %d (%s): %s" % (code, name, detail))


def _check(code, ctx=None):
    if code != _lib.OK:
        msg = _lib.lib().trhip_last_error(ctx).decode(errors="replace")
        raise TrhipError(code, msg)


def dtype_code(dt):
    return BY_NAME[dt] if isinstance(dt, str) else int(dt)


def CheckQuantScales(dt, raw):
    """Index of the first block with a NaN/Inf fp16 scale, or -1 (tensor/quant.go:108-128)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    bad = ctypes.c_int64()
    _check(_lib.lib().trhip_check_quant_scales(dtype_code(dt), raw.ctypes.data_as(P), raw.nbytes, ctypes.byref(bad)))
    return bad.value


def device_count():
    n = ctypes.c_int()
    _lib.lib().trhip_device_count(ctypes.byref(n))
    return n.value


class DeviceBuffer:
    """Device allocation on one context (Storage analogue for fp32 activations/outputs)."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = P()
        _check(_lib.lib().trhip_alloc(ctx.h, self.nbytes, ctypes.byref(p)), ctx.h)
        self.ptr = p.value

    def addr(self, byte_offset=0):
        return P(self.ptr + byte_offset)

    def upload(self, arr, byte_offset=0):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes + byte_offset <= self.nbytes
        _check(_lib.lib().trhip_h2d_async(self.ctx.h, self.addr(byte_offset), arr.ctypes.data_as(P), arr.nbytes), self.ctx.h)
        self.ctx.sync()  # the host array may be temporary
        return self

    def download(self, dtype, count, byte_offset=0):
        out = np.empty(count, dtype=dtype)
        _check(_lib.lib().trhip_d2h(self.ctx.h, out.ctypes.data_as(P), self.addr(byte_offset), out.nbytes), self.ctx.h)
        return out

    def fill(self, value_byte, nbytes=None):
        _check(_lib.lib().trhip_memset_async(self.ctx.h, self.addr(), value_byte, self.nbytes if nbytes is None else nbytes), self.ctx.h)

    def free(self):
        if self.ptr:
            _lib.lib().trhip_free(self.ctx.h, P(self.ptr))
            self.ptr = 0


class Context:
    """One device and one in-order stream (trhip_ctx)."""

    def __init__(self, device=0):
        h = P()
        _check(_lib.lib().trhip_init(device, ctypes.byref(h)))
        self.h = h
        self.device = device

    def alloc(self, nbytes):
        return DeviceBuffer(self, nbytes)

    def to_device(self, arr):
        arr = np.ascontiguousarray(arr)
        return self.alloc(max(arr.nbytes, 1)).upload(arr)

    def sync(self):
        _check(_lib.lib().trhip_sync(self.h), self.h)

    def event(self):
        e = P()
        _check(_lib.lib().trhip_event_create(self.h, ctypes.byref(e)), self.h)
        return e

    def record(self, ev):
        _check(_lib.lib().trhip_event_record(self.h, ev), self.h)

    def host_alloc(self, nbytes):
        """Page-locked host memory as a numpy uint8 array (trhip_host_alloc); free with host_free."""
        p = P()
        _check(_lib.lib().trhip_host_alloc(self.h, max(int(nbytes), 1), ctypes.byref(p)), self.h)
        arr = np.ctypeslib.as_array((ctypes.c_uint8 * max(int(nbytes), 1)).from_address(p.value))[:int(nbytes)]
        return arr, p

    def host_free(self, p):
        _check(_lib.lib().trhip_host_free(self.h, p), self.h)

    def set_launch_shape(self, knob, a=0, b=0, c=0, d=0):
        """Force a launch shape (tests and tuning; all zero restores the built-in choice)."""
        _check(_lib.lib().trhip_set_launch_shape(self.h, knob, a, b, c, d), self.h)

    def read_probe(self, buf, nbytes=None):
        """Read nbytes of buf once on the device (the single-launch streaming-read ceiling; writes nothing)."""
        _check(_lib.lib().trhip_read_probe(self.h, buf.addr(), buf.nbytes if nbytes is None else nbytes), self.h)

    @staticmethod
    def elapsed_ms(a, b):
        ms = ctypes.c_float()
        _check(_lib.lib().trhip_event_elapsed_ms(a, b, ctypes.byref(ms)))
        return ms.value

    def close(self):
        """Destroy the context; it is refused (and kept) while stores or graphs made on it are alive."""
        if self.h:
            code = _lib.lib().trhip_destroy(self.h)
            if code == _lib.OK:
                self.h = None
            return code
        return _lib.OK


class QuantWeight:
    """Device-resident GGUF weight [N, K] (trhip_wstore)."""

    def __init__(self, ctx, dt, raw, N, K, zero=False):
        self.ctx = ctx
        self.dt = dtype_code(dt)
        self.N, self.K = int(N), int(K)
        if raw is None:  # filled by the caller (Concat) or zeroed
            self.h = P()
            if zero:
                _check(_lib.lib().trhip_wstore_create_zero(ctx.h, self.dt, self.N, self.K, ctypes.byref(self.h)), ctx.h)
            return
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        h = P()
        _check(_lib.lib().trhip_wstore_create(ctx.h, self.dt, raw.ctypes.data_as(P), raw.nbytes, self.N, self.K, ctypes.byref(h)), ctx.h)
        ctx.sync()  # the host bytes may be released after this returns
        self.h = h

    @staticmethod
    def Concat(parts):
        """One store with the rows of `parts` in order (a merged layer: [gate | up], [q | k | v])."""
        ctx = parts[0].ctx
        w = QuantWeight(ctx, parts[0].dt, None, sum(p.N for p in parts), parts[0].K)
        hs = (P * len(parts))(*[p.h for p in parts])
        _check(_lib.lib().trhip_wstore_concat(ctx.h, hs, len(parts), ctypes.byref(w.h)), ctx.h)
        return w

    def ToRaw(self, row0=0, rows=None):
        rows = self.N - row0 if rows is None else rows
        elems, size = BLOCK[self.dt]
        out = np.empty(rows * (self.K // elems) * size, dtype=np.uint8)
        _check(_lib.lib().trhip_wstore_to_raw(self.ctx.h, self.h, row0, rows, out.ctypes.data_as(P)), self.ctx.h)
        return out

    def device_bytes(self):
        n = ctypes.c_size_t()
        _check(_lib.lib().trhip_wstore_info(self.h, None, None, None, ctypes.byref(n)))
        return n.value

    def release(self):
        if self.h:
            _lib.lib().trhip_wstore_destroy(self.h)
            self.h = None


def _ptr(x):
    if isinstance(x, DeviceBuffer):
        return x.addr()
    if isinstance(x, tuple):  # (buffer, byte_offset)
        return x[0].addr(x[1])
    return P(int(x))


class QuantBackend:
    """The quantized-matmul slice of the reference's Backend, on one MI355X context."""

    def __init__(self, device=0):
        self.ctx = Context(device)

    def FromQuantized(self, dt, raw, N, K):
        return QuantWeight(self.ctx, dt, raw, N, K)

    def NewQuantStorage(self, dt, N, K):
        """Zeroed quantized storage: every element opens to +0 (tensor/quant.go:408-427)."""
        return QuantWeight(self.ctx, dt, None, N, K, zero=True)

    def Gemm(self, M, N, K, a, w, c, row0=0, mode=MODE_EXACT):
        _check(_lib.lib().trhip_gemm_q(self.ctx.h, w.h, row0, N, _ptr(a), _ptr(c), M, K, 1, mode), self.ctx.h)

    def GemmSet(self, M, N, K, a, w, c, row0=0, mode=MODE_EXACT):
        _check(_lib.lib().trhip_gemm_q(self.ctx.h, w.h, row0, N, _ptr(a), _ptr(c), M, K, 0, mode), self.ctx.h)

    def GemmTyped(self, M, N, K, a, atype, w, c, ctype, row0=0, accumulate=False, mode=MODE_EXACT):
        """Gemm / GemmSet with 16-bit activations or outputs (atype, ctype: F32, F16, BF16): a widened to fp32, the
        fp32 product, c rounded once (gpu/backend_quant.go:41-45)."""
        _check(_lib.lib().trhip_gemm_q_typed(self.ctx.h, w.h, row0, N, _ptr(a), atype, _ptr(c), ctype, M, K,
                                             1 if accumulate else 0, mode), self.ctx.h)

    def GemmActQuant(self, M, N, K, a, w, c, row0=0, accumulate=True, mode=MODE_EXACT):
        """ActQuantGemmer.GemmActQuant (tensor/matmul.go:59-61); mode=MODE_FAST fuses the fp32 epilogue over the same
        exact integer block sums (trhip_gemm_q_actq_mode)."""
        if mode == MODE_EXACT:
            _check(_lib.lib().trhip_gemm_q_actq(self.ctx.h, w.h, row0, N, _ptr(a), _ptr(c), M, K, 1 if accumulate else 0),
                   self.ctx.h)
        else:
            _check(_lib.lib().trhip_gemm_q_actq_mode(self.ctx.h, w.h, row0, N, _ptr(a), _ptr(c), M, K,
                                                     1 if accumulate else 0, mode), self.ctx.h)

    def SwiGLU(self, gu, M, I, out):
        """out[m, i] = silu(gu[m, i]) * gu[m, I + i] (lib/layers.tr:223 on a merged [gate | up] output)."""
        _check(_lib.lib().trhip_swiglu(self.ctx.h, _ptr(gu), M, I, _ptr(out)), self.ctx.h)

    def GemmSwiGLU(self, M, K, a, w, out, mode=MODE_EXACT):
        """SwiGLU of x @ w^T for a merged [gate | up] store of 2I rows; out is [M, I]."""
        _check(_lib.lib().trhip_gemm_q_swiglu(self.ctx.h, w.h, _ptr(a), _ptr(out), M, K, mode), self.ctx.h)

    def OpenQuant(self, out, w, offset=0, n=None):
        n = w.N * w.K - offset if n is None else n
        _check(_lib.lib().trhip_open_q(self.ctx.h, w.h, offset, n, _ptr(out)), self.ctx.h)

    def Embedding(self, out, w, idx):
        idx = np.ascontiguousarray(idx, dtype=np.int64)
        _check(_lib.lib().trhip_embedding_q(self.ctx.h, w.h, idx.ctypes.data_as(P), idx.size, _ptr(out)), self.ctx.h)

    def QuantizeQ8(self, x, M, K, blk, q, d, bs):
        _check(_lib.lib().trhip_quantize_q8(self.ctx.h, _ptr(x), M, K, blk, _ptr(q), _ptr(d), _ptr(bs)), self.ctx.h)

    def close(self):
        self.ctx.close()
