"""ctypes binding of libtrhip (include/trhip.h).

The library is loaded from this package directory only; there is no fallback. A missing or
stale build raises ImportError with the path, so nothing can silently run on the CPU.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtrhip.so")

P = ctypes.c_void_p
I64 = ctypes.c_int64
SZ = ctypes.c_size_t
INT = ctypes.c_int

# (name, restype, argtypes) for every entry point declared in include/trhip.h
SIGNATURES = [
    ("trhip_strerror", ctypes.c_char_p, [INT]),
    ("trhip_last_error", ctypes.c_char_p, [P]),
    ("trhip_version", INT, []),
    ("trhip_device_count", INT, [ctypes.POINTER(INT)]),
    ("trhip_init", INT, [INT, ctypes.POINTER(P)]),
    ("trhip_destroy", INT, [P]),
    ("trhip_stream", P, [P]),
    ("trhip_alloc", INT, [P, SZ, ctypes.POINTER(P)]),
    ("trhip_free", INT, [P, P]),
    ("trhip_h2d_async", INT, [P, P, P, SZ]),
    ("trhip_d2h", INT, [P, P, P, SZ]),
    ("trhip_memset_async", INT, [P, P, INT, SZ]),
    ("trhip_sync", INT, [P]),
    ("trhip_host_alloc", INT, [P, SZ, ctypes.POINTER(P)]),
    ("trhip_host_free", INT, [P, P]),
    ("trhip_event_create", INT, [P, ctypes.POINTER(P)]),
    ("trhip_event_record", INT, [P, P]),
    ("trhip_event_elapsed_ms", INT, [P, P, ctypes.POINTER(ctypes.c_float)]),
    ("trhip_event_destroy", INT, [P]),
    ("trhip_graph_begin", INT, [P]),
    ("trhip_graph_end", INT, [P, ctypes.POINTER(P)]),
    ("trhip_graph_launch", INT, [P, P]),
    ("trhip_graph_destroy", INT, [P]),
    ("trhip_check_quant_scales", INT, [INT, P, SZ, ctypes.POINTER(I64)]),
    ("trhip_wstore_create", INT, [P, INT, P, SZ, I64, I64, ctypes.POINTER(P)]),
    ("trhip_wstore_create_zero", INT, [P, INT, I64, I64, ctypes.POINTER(P)]),
    ("trhip_wstore_destroy", INT, [P]),
    ("trhip_wstore_info", INT, [P, ctypes.POINTER(INT), ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(SZ)]),
    ("trhip_wstore_to_raw", INT, [P, P, I64, I64, P]),
    ("trhip_wstore_concat", INT, [P, P, INT, ctypes.POINTER(P)]),
    ("trhip_gemm_q", INT, [P, P, I64, I64, P, P, I64, I64, INT, INT]),
    ("trhip_gemm_q_typed", INT, [P, P, I64, I64, P, INT, P, INT, I64, I64, INT, INT]),
    ("trhip_gemm_q_actq", INT, [P, P, I64, I64, P, P, I64, I64, INT]),
    ("trhip_gemm_q_actq_noalloc", INT, [P, P, I64, I64, P, P, I64, I64, INT]),
    ("trhip_gemm_q_actq_mode", INT, [P, P, I64, I64, P, P, I64, I64, INT, INT]),
    ("trhip_open_q", INT, [P, P, I64, I64, P]),
    ("trhip_read_probe", INT, [P, P, I64]),
    ("trhip_mfma_probe", INT, [P, INT, INT, I64]),
    ("trhip_prefill_probe", INT, [P, INT, I64, I64, I64]),
    ("trhip_embedding_q", INT, [P, P, P, I64, P]),
    ("trhip_quantize_q8", INT, [P, P, I64, I64, INT, P, P, P]),
    ("trhip_swiglu", INT, [P, P, I64, I64, P]),
    ("trhip_gemm_q_swiglu", INT, [P, P, P, P, I64, I64, INT]),
    ("trhip_set_launch_shape", INT, [P, INT, INT, INT, INT, INT]),
]

# Status codes and enums (include/trhip.h)
OK, ERR_INVALID, ERR_OOM, ERR_HIP, ERR_LAUNCH, ERR_UNSUPPORTED, ERR_NO_DEVICE, ERR_BAD_SCALE = range(8)
Q8, Q4, Q4K, Q6K = 1, 2, 3, 4
MODE_EXACT, MODE_FAST = 0, 1
F32, F16, BF16 = 0, 1, 2
KNOB_KL, KNOB_FAST_Q4K, KNOB_EXACT_ROWS, KNOB_EXACT_LANES, KNOB_ACTQ_TM, KNOB_ROWS16, KNOB_KL_GRID = 1, 2, 3, 4, 5, 6, 7


def load(path=LIB_PATH):
    if not os.path.exists(path):
        raise ImportError("libtrhip.so is not built at %s (run __graft_entry__.build())" % path)
    lib = ctypes.CDLL(path)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB
