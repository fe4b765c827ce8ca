"""ctypes declarations for libredshift_hip.

``load_library`` mirrors the reference's loader (qvelox/runtime.py:6-22): same
function name, same five ``qv_test_*`` signatures, and it raises if any of
them is missing.  It additionally declares the device ABI of include/runtime.h.
The default path is this package's in-tree build, ``lib/libredshift_hip.so``;
a missing build is an error (there is no fallback implementation).
"""
import ctypes as ct
from pathlib import Path

DEFAULT_LIBRARY = Path(__file__).resolve().parent / 'lib' / 'libredshift_hip.so'

QV_F16 = 1
QV_BF16 = 2
QV_F32 = 3

# The reference's validation ABI (qvelox/runtime.py:13-17).
TEST_SIGNATURES = {
    'qv_test_mm': [ct.c_void_p] * 3 + [ct.c_int] * 4,
    'qv_test_mm_fast': [ct.c_void_p] * 3 + [ct.c_int] * 4,
    'qv_test_norm': [ct.c_void_p] * 3 + [ct.c_int] * 2 + [ct.c_float],
    'qv_test_delta': [ct.c_void_p] * 11 + [ct.c_int] * 4 + [ct.c_float],
    'qv_test_attention': [ct.c_void_p] * 8 + [ct.c_int] * 2 + [ct.c_float],
}

# Model session ABI (qvelox/runtime.py:37-51): exported, returns -1 here.
SESSION_SIGNATURES = {
    'qv_create': [ct.POINTER(ct.c_void_p), ct.c_char_p, ct.c_int, ct.c_float],
    'qv_upload': [ct.c_void_p, ct.c_int, ct.c_uint64, ct.c_uint64],
    'qv_evaluate': [ct.c_void_p, ct.POINTER(ct.c_int), ct.c_int, ct.POINTER(ct.c_float)],
    'qv_verify': [ct.c_void_p, ct.POINTER(ct.c_int), ct.c_int, ct.POINTER(ct.c_float)],
    'qv_commit': [ct.c_void_p, ct.c_int],
    'qv_advance': [ct.c_void_p, ct.POINTER(ct.c_int), ct.c_int, ct.POINTER(ct.c_int)],
    'qv_position': [ct.c_void_p, ct.POINTER(ct.c_int)],
    'qv_reset': [ct.c_void_p], 'qv_checkpoint': [ct.c_void_p], 'qv_restore': [ct.c_void_p],
}

_P, _I, _F, _U64 = ct.c_void_p, ct.c_int, ct.c_float, ct.c_uint64
DEVICE_SIGNATURES = {
    'qv_kv_bytes': [ct.POINTER(_U64), _I, _I, _I],
    'qv_kv_pack': [_P] * 4 + [_I] * 5 + [_P],
    'qv_kv_unpack': [_P] * 4 + [_I] * 5 + [_P],
    'qv_kv_copy': [_P] * 4 + [_I] * 5 + [_P],
    'qv_attention_workspace': [ct.POINTER(_U64)] + [_I] * 5,
    'qv_attention': [_P] * 4 + [_I] * 8 + [_F, _P, _U64, _P],
    'qv_attention_split': [_P] * 3 + [_I] * 7 + [_F, _P, _U64, _P],
    'qv_attention_combine': [_P] + [_I] * 7 + [_P, _U64, _P],
    'qv_attention_noalloc': [_P] * 4 + [_I] * 8 + [_F, _P],
    'qv_attention_precise_workspace': [ct.POINTER(_U64)] + [_I] * 5,
    'qv_attention_precise': [_P] * 4 + [_I] * 6 + [_F, _P, _U64, _P],
    'qv_attention_fused_workspace': [ct.POINTER(_U64), _I, _I],
    'qv_attention_fused': [_P] * 8 + [_I] * 3 + [_F, _P, _U64, _P],
}


def load_library(path=None):
    """Load libredshift_hip and declare its C ABI (qvelox/runtime.py:6-22)."""
    path = Path(path) if path is not None else DEFAULT_LIBRARY
    if not path.exists():
        raise RuntimeError(f'{path} is missing: build it with `python -m redshift_amd.build`')
    lib = ct.CDLL(str(path.resolve()))
    lib.qv_error.argtypes = []
    lib.qv_error.restype = ct.c_char_p
    for table in (TEST_SIGNATURES, SESSION_SIGNATURES, DEVICE_SIGNATURES):
        for name, signature in table.items():
            function = getattr(lib, name)
            function.argtypes = signature
            function.restype = ct.c_int
    lib.qv_destroy.argtypes = [ct.c_void_p]
    lib.qv_destroy.restype = None
    return lib


_LIBRARY = None


def library():
    """The process-wide handle of the in-tree library (loaded on first use)."""
    global _LIBRARY
    if _LIBRARY is None:
        _LIBRARY = load_library()
    return _LIBRARY


def check(lib, code):
    """Raise RuntimeError with qv_error() when an entry point returned -1."""
    if code:
        raise RuntimeError(lib.qv_error().decode('utf-8', errors='replace'))
