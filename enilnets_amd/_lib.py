"""ctypes binding of libenilnets_amd.so (the C ABI in include/enilnets_amd.h).

The library is loaded lazily on first use.  There is no fallback: if the
shared library is missing or no gfx950 device is visible, calls raise.
"""

import ctypes
import os
import threading
from ctypes import (POINTER, c_char, c_char_p, c_double, c_float, c_int, c_int8,
                    c_int32, c_int64, c_size_t, c_void_p)
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libenilnets_amd.so"

# status codes (include/enilnets_amd.h)
OK = 0
ERR_INVALID = 1
ERR_RUNTIME = 2
ERR_NO_DEVICE = 3
ERR_UNSUPPORTED = 4

F32 = 0
F64 = 1
SYMMETRIC = 0
ASYMMETRIC = 1
W8_FP32 = 0
W8_BF16 = 1
AQ_NONE = 0
AQ_F32 = 1
AQ_F64 = 2

ACTIVATIONS = {
    "linear": 0, "relu": 1, "leakyrelu": 2, "elu": 3, "selu": 4, "gelu": 5,
    "swish": 6, "mish": 7, "sigmoid": 8, "tanh": 9, "softplus": 10, "softmax": 11,
}


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", c_char * 128),
        ("arch", c_char * 64),
        ("device", c_int),
        ("compute_units", c_int),
        ("clock_khz", c_int),
        ("memory_clock_khz", c_int),
        ("memory_bus_width", c_int),
        ("l2_bytes", c_int),
        ("lds_bytes_per_block", c_int),
        ("wavefront_size", c_int),
        ("global_memory_bytes", ctypes.c_longlong),
    ]


_P = c_void_p
#: Every exported function: name -> (restype, argtypes).
SIGNATURES = {
    "enq_abi_version": (c_int, []),
    "enq_init": (c_int, [c_int]),
    "enq_get_device_info": (c_int, [POINTER(DeviceInfo)]),
    "enq_synchronize": (c_int, []),
    "enq_last_error": (c_char_p, []),
    "enq_get_stream": (c_int, [POINTER(c_void_p)]),
    "enq_set_stream": (c_int, [_P]),
    "enq_graph_begin": (c_int, []),
    "enq_graph_end": (c_int, [_P]),
    "enq_graph_launch": (c_int, [_P]),
    "enq_graph_destroy": (c_int, [_P]),
    "enq_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "enq_free": (c_int, [_P]),
    "enq_release_cached_memory": (c_int, []),
    "enq_copy_to_device": (c_int, [_P, _P, c_size_t]),
    "enq_copy_to_host": (c_int, [_P, _P, c_size_t]),
    "enq_copy_on_device": (c_int, [_P, _P, c_size_t]),
    "enq_event_create": (c_int, [POINTER(c_void_p)]),
    "enq_event_destroy": (c_int, [_P]),
    "enq_event_record": (c_int, [_P]),
    "enq_event_elapsed_ms": (c_int, [_P, _P, POINTER(c_float)]),
    "enq_minmax": (c_int, [c_int, _P, c_int64, c_int64, c_int64, _P, _P]),
    "enq_compute_scale": (c_int, [c_int, _P, _P, c_int64, c_int, c_int, _P, _P]),
    "enq_quantize": (c_int, [c_int, _P, c_int64, c_int64, c_int64, _P, _P, c_int, c_int, _P]),
    "enq_quantize_codes_i8": (c_int, [c_int, _P, c_int64, c_int64, c_int64, _P, _P, c_int,
                                      c_int, _P]),
    "enq_dequantize": (c_int, [c_int, _P, c_int64, c_int64, c_int64, _P, _P, _P]),
    "enq_fake_quantize": (c_int, [c_int, _P, c_int64, c_int64, c_int64, _P, _P, c_int, c_int,
                                  _P]),
    "enq_quantize_tensor": (c_int, [c_int, _P, c_int64, c_int64, c_int64, c_int, c_int, _P, _P,
                                    _P, _P, _P]),
    "enq_quantize_rows_i8": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "enq_dequantize_i8": (c_int, [c_int, _P, c_int64, c_int64, c_int64, _P, _P]),
    "enq_error_stats": (c_int, [c_int, _P, _P, c_int64, POINTER(c_double)]),
    "enq_order_stats": (c_int, [c_int, _P, c_int64, POINTER(c_int64), c_int, _P]),
    "enq_dense_w8": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float, c_float,
                             c_int, _P, _P]),
    "enq_split_planes": (c_int, [_P, c_int64, c_int64, c_int, _P]),
    "enq_gemm_w8_planes": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float,
                                   c_float, c_int, _P, _P]),
    "enq_split_f16f8": (c_int, [_P, c_int64, c_int64, _P]),
    "enq_gemm_w8_f16f8": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float,
                                  c_float, _P, _P]),
    "enq_dense_w8_ffn": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float,
                                 c_float, _P, _P, _P, c_int64, _P, c_int, c_float, c_float,
                                 c_int, _P]),
    "enq_f16f8_bound": (c_int, [_P, c_int64, c_int64, _P, _P, c_int, c_float, c_float, _P]),
    "enq_dense_w8_noalloc": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float,
                                     c_float, c_int, _P, _P]),
    "enq_gemm_w8a8": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int, c_float,
                              c_float, _P, _P]),
    "enq_dense_w8a8": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float,
                               c_float, _P, _P]),
    "enq_dense_w8_aq": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, _P, c_int, c_float,
                                c_float, c_int, c_int, c_double, c_double, c_float, c_float,
                                _P, _P]),
    "enq_dense_w8a8_static": (c_int, [_P, c_int64, c_int64, c_int, c_double, c_double, c_float,
                                      c_float, _P, _P, _P, c_int64, _P, c_int, c_float, c_float,
                                      _P, _P]),
    "enq_code_row_sums": (c_int, [_P, c_int64, c_int64, _P]),
    "enq_act_quant": (c_int, [_P, c_int64, c_int, c_double, c_double, c_float, c_float, _P]),
    "enq_layernorm": (c_int, [_P, c_int64, c_int64, _P, _P, c_float, _P]),
    "enq_add": (c_int, [_P, _P, c_int64, _P]),
    "enq_attention": (c_int, [_P, c_int64, _P, c_int64, _P, c_int64, c_int64, c_int64, c_int,
                              c_int, c_int, c_int, c_int64, _P, c_int64]),
    "enq_attention_kv": (c_int, [_P, c_int64, c_int64, c_int64, c_int64, _P, c_int64, _P,
                                 c_int64, c_int64, c_int64, c_int64, c_int64, c_int, c_int,
                                 c_int, c_int, c_int64, _P, c_int64]),
    "enq_add_bcast": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "enq_copy_rows": (c_int, [_P, c_int64, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64,
                              c_int64]),
    "enq_moe_w8": (c_int, [_P, c_int64, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                           c_int64, c_int64, c_int, c_int, c_float, c_float, _P, c_int, _P, _P,
                           _P, _P]),
}

_lock = threading.RLock()
_lib = None
_initialised = False

_EXC = {
    ERR_INVALID: ValueError,
    ERR_RUNTIME: RuntimeError,
    ERR_NO_DEVICE: RuntimeError,
    ERR_UNSUPPORTED: NotImplementedError,
}


def load() -> ctypes.CDLL:
    """Load the shared library and declare every signature (no device use)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m enilnets_amd.csrc.build` "
                "(enilnets_amd has no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def check(status: int) -> None:
    """Raise the Python exception matching a non-zero status."""
    if status == OK:
        return
    msg = load().enq_last_error().decode(errors="replace")
    raise _EXC.get(status, RuntimeError)(msg)


def lib() -> ctypes.CDLL:
    """The library, initialised on the device named by ENILNETS_AMD_DEVICE
    (default 0)."""
    global _initialised
    handle = load()
    if not _initialised:
        with _lock:
            if not _initialised:
                check(handle.enq_init(int(os.environ.get("ENILNETS_AMD_DEVICE", "0"))))
                _initialised = True
    return handle


def call(name: str, *args) -> None:
    """Call an ABI function and raise on failure."""
    check(getattr(lib(), name)(*args))


def device_info() -> DeviceInfo:
    info = DeviceInfo()
    call("enq_get_device_info", ctypes.byref(info))
    return info


def synchronize() -> None:
    call("enq_synchronize")
