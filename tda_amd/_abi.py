"""ctypes binding of libtda_hip.so (declared in include/tda.h).

The structs below mirror tda_fwd_args / tda_bwd_args field for field (ctypes applies the
same natural alignment as the C compiler).  The library's ABI version is checked at load
time.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(HERE, "libtda_hip.so")

ABI_VERSION = 7
DTYPE_F32 = 0
DTYPE_BF16 = 1

OK = 0
ERR_NULL_POINTER = -1
ERR_SHAPE = -2
ERR_HEAD_DIM = -3
ERR_DTYPE = -4
ERR_LAYOUT = -5
ERR_POWER = -6
ERR_BRANCHES = -7
ERR_WORKSPACE = -8
ERR_ABI = -9
ERR_CAUSAL = -10
ERR_NORMS = -11
ERR_OFFSET = -12
ERR_SCRATCH = -13
ERR_HIP = -100
NOALLOC_SCRATCH_BYTES = 16 << 20


class TdaTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("stride", ctypes.c_int64 * 4)]


_COMMON = [
    ("abi_version", ctypes.c_int32),
    ("dtype", ctypes.c_int32),
    ("branches", ctypes.c_int32),
    ("normalize", ctypes.c_int32),
    ("causal", ctypes.c_int32),
    ("relu_power", ctypes.c_float),
    ("batch", ctypes.c_int64),
    ("heads", ctypes.c_int64),
    ("seq_len", ctypes.c_int64),
    ("head_dim", ctypes.c_int64),
]


class TdaFwdArgs(ctypes.Structure):
    _fields_ = _COMMON + [
        ("q1", TdaTensor), ("k1", TdaTensor), ("q2", TdaTensor), ("k2", TdaTensor),
        ("v", TdaTensor), ("out", TdaTensor),
        ("beta", ctypes.c_void_p), ("lambda_param", ctypes.c_void_p),
        ("norms", ctypes.c_void_p), ("occupancy", ctypes.c_void_p), ("stats", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("seq_len_kv", ctypes.c_int64), ("q_offset", ctypes.c_int64),
        ("pairs", ctypes.c_void_p),
        ("zero", ctypes.c_void_p), ("zero_bytes", ctypes.c_uint64),
    ]


class TdaBwdArgs(ctypes.Structure):
    _fields_ = _COMMON + [
        ("q1", TdaTensor), ("k1", TdaTensor), ("q2", TdaTensor), ("k2", TdaTensor),
        ("v", TdaTensor), ("dout", TdaTensor),
        ("dq1", TdaTensor), ("dk1", TdaTensor), ("dq2", TdaTensor), ("dk2", TdaTensor),
        ("dv", TdaTensor),
        ("beta", ctypes.c_void_p), ("lambda_param", ctypes.c_void_p),
        ("dbeta", ctypes.c_void_p), ("dlambda", ctypes.c_void_p),
        ("norms", ctypes.c_void_p), ("occupancy", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stats", ctypes.c_void_p),
        ("seq_len_kv", ctypes.c_int64), ("q_offset", ctypes.c_int64),
        ("pairs", ctypes.c_void_p),
        ("grads_zeroed", ctypes.c_int32),
    ]


# Every function include/tda.h declares: name -> (restype, argtypes)
SIGNATURES = {
    "tda_abi_version": (ctypes.c_int32, []),
    "tda_error_string": (ctypes.c_char_p, [ctypes.c_int32]),
    "tda_last_hip_error": (ctypes.c_int32, []),
    "tda_validate_fwd": (ctypes.c_int32, [ctypes.POINTER(TdaFwdArgs)]),
    "tda_validate_bwd": (ctypes.c_int32, [ctypes.POINTER(TdaBwdArgs)]),
    "tda_occupancy_words": (ctypes.c_size_t, [ctypes.c_int64] * 3 + [ctypes.c_int32]),
    "tda_norms_floats": (ctypes.c_size_t, [ctypes.c_int64] * 3 + [ctypes.c_int32]),
    "tda_fwd_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3 + [ctypes.c_int32]),
    "tda_occupancy_words_kv": (ctypes.c_size_t, [ctypes.c_int64] * 4 + [ctypes.c_int32]),
    "tda_norms_floats_kv": (ctypes.c_size_t, [ctypes.c_int64] * 4 + [ctypes.c_int32]),
    "tda_fwd_workspace_bytes_kv": (ctypes.c_size_t, [ctypes.c_int64] * 4 + [ctypes.c_int32]),
    "tda_fwd_workspace_bytes_for": (ctypes.c_size_t, [ctypes.POINTER(TdaFwdArgs)]),
    "tda_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 4),
    "tda_pair_words": (ctypes.c_size_t, [ctypes.c_int64] * 3 + [ctypes.c_int32]),
    "tda_fwd": (ctypes.c_int32, [ctypes.POINTER(TdaFwdArgs), ctypes.c_void_p]),
    "tda_bwd": (ctypes.c_int32, [ctypes.POINTER(TdaBwdArgs), ctypes.c_void_p]),
    "tda_fwd_noalloc": (ctypes.c_int32, [ctypes.POINTER(TdaFwdArgs), ctypes.c_void_p]),
    "tda_time_next_call": (ctypes.c_int32, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int32]),
    "tda_timed_launches": (ctypes.c_int32, []),
    "tda_timed_launch_name": (ctypes.c_char_p, [ctypes.c_int32]),
}

_lock = threading.Lock()
_lib = None


def lib_path() -> str:
    return os.environ.get("TDA_HIP_LIB", DEFAULT_LIB)


def load(path: str | None = None):
    """Load (once) and return the library.  Raises RuntimeError when it is missing: there is
    no CPU fallback."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or lib_path()
        if not os.path.exists(p):
            raise RuntimeError(
                f"tda_amd: native library {p} is missing; build it with "
                "`python -m tda_amd.build` (hipcc, gfx950). There is no CPU fallback.")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.tda_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"tda_amd: {p} has ABI version {v}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


class TdaError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def check(code: int, what: str) -> None:
    """Map a C-ABI return code to an exception: argument errors -> ValueError,
    launch failures -> RuntimeError."""
    if code == OK:
        return
    lib = load()
    msg = f"{what}: {lib.tda_error_string(code).decode()} (code {code})"
    if code == ERR_HIP:
        raise TdaError(code, f"{msg}; hipError_t {lib.tda_last_hip_error()}")
    raise ValueError(msg)
