"""ctypes binding of liblq.so (include/lq.h).  The product path has no fallback: if the library is missing or a call
fails, this raises."""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liblq.so")
ABI_VERSION = 5
SCHED_INTS = 512           # include/lq.h: LQ_SCHED_INTS

c_void_p, c_int, c_float, c_ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong


class LqState(ctypes.Structure):
    _fields_ = [("ssm", c_void_p), ("slot_stride", c_ll), ("Kbuf", c_void_p), ("Ubuf", c_void_p),
                ("Wbuf", c_void_p), ("Pbuf", c_void_p), ("Gbuf", c_void_p), ("hcnt", c_void_p),
                ("NS", c_int), ("HV", c_int), ("H", c_int), ("K", c_int), ("V", c_int), ("L", c_int), ("R", c_int),
                ("ctl", c_void_p), ("qmax", c_float), ("sched", c_void_p)]


class LqStepIO(ctypes.Structure):
    _fields_ = [("mixed", c_void_p), ("a", c_void_p), ("b", c_void_p), ("A_log", c_void_p), ("dt_bias", c_void_p),
                ("idx", c_void_p), ("out", c_void_p), ("N", c_int), ("scale", c_float)]


class LqConv(ctypes.Structure):
    _fields_ = [("state", c_void_p), ("weight", c_void_p), ("bias", c_void_p), ("slot_stride", c_ll),
                ("ch_stride", c_ll), ("tap_stride", c_ll), ("W", c_int), ("silu", c_int), ("NS", c_int)]


# exported symbol -> (restype, argtypes); must match include/lq.h
SIGNATURES = {
    "lq_abi_version": (c_int, []),
    "lq_gdn_step": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), c_void_p]),
    "lq_gdn_step_conv": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), ctypes.POINTER(LqConv), c_void_p]),
    "lq_kda_step": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), c_float, c_void_p]),
    "lq_kda_decode": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), c_float, c_void_p, c_void_p]),
    "lq_gdn_decode": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), ctypes.POINTER(LqConv), c_void_p,
                              c_void_p]),
    "lq_gdn_decode_deferred": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), ctypes.POINTER(LqConv),
                                       c_void_p, c_void_p]),
    "lq_flush": (c_int, [ctypes.POINTER(LqState), c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "lq_quantize": (c_int, [ctypes.POINTER(LqState), c_void_p, c_void_p, c_int, c_float, c_void_p]),
    "lq_dequant": (c_int, [ctypes.POINTER(LqState), c_void_p, c_int, c_float, c_void_p]),
    "lq_kda_dequant": (c_int, [ctypes.POINTER(LqState), c_void_p, c_int, c_float, c_void_p]),
    "lq_kda_checkpoint": (c_int, [ctypes.POINTER(LqState), c_void_p, c_void_p, c_int, c_float, c_void_p]),
    "lq_lowrank": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "lq_conv_update": (c_int, [ctypes.POINTER(LqConv), c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "lq_dense_step": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, ctypes.POINTER(LqStepIO),
                              c_void_p]),
    "lq_decode_noalloc": (c_int, [ctypes.POINTER(LqState), ctypes.POINTER(LqStepIO), c_void_p, c_int, c_float,
                                  c_void_p]),
}

_LIB = [None]


def lib():
    """The loaded liblq.so (raises if it has not been built)."""
    if _LIB[0] is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("liblq.so is missing (%s): build it with `python -m leapquant_amd.build`" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        v = L.lq_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError("liblq.so ABI %d, expected %d: rebuild it" % (v, ABI_VERSION))
        _LIB[0] = L
    return _LIB[0]


_ERR = {-1: "bad argument (unsupported shape / size / pointer)", -2: "HIP launch error",
        -3: "more (row, head) pairs than the static due list of lq_decode_noalloc holds (N * HV <= 65536)"}


def check(rc, what):
    if rc != 0:
        raise RuntimeError("%s failed: %s (status %d)" % (what, _ERR.get(rc, "unknown"), rc))
