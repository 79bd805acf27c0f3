"""ctypes binding of the C ABI in include/rsfa.h (librsfa.so).

The library holds the gfx950 kernels; there is no other compute path.  Loading
fails loudly when the library has not been built.
"""
import ctypes
import os
import threading

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "librsfa.so")

ABI_VERSION = 6

# rsfa_status
OK = 0
E_NULL = -1
E_SHAPE = -2
E_HEADDIM = -3
E_DTYPE = -4
E_TILE = -5
E_ALIGN = -6
E_DEVICE = -7
E_LAUNCH = -8
E_ABI = -9
E_WORKSPACE = -10
E_SCRATCH = -11

# rsfa_dtype
DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F16_V8E5M2 = 2  # q, k, o float16; v float8_e5m2

# flags
FLAG_STATIC_SCHEDULE = 0x1
FLAG_CAUSAL_SPLIT = 0x2
FLAG_EXACT_TILE = 0x4
FLAG_TILE_HINT = 0x8
FLAG_SINGLE_BLOCKS = 0x10

# rsfa_attention_fwd_noalloc's fixed workspace
NOALLOC_WORKSPACE_BYTES = 16 << 20

# Every symbol include/rsfa.h declares, with (restype, argtypes).
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_PI32 = ctypes.POINTER(ctypes.c_int32)


class FwdArgs(ctypes.Structure):
    """Mirror of struct rsfa_fwd_args."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("dtype", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("z", ctypes.c_int64),
        ("h", ctypes.c_int64),
        ("n_ctx", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_stride", ctypes.c_int64 * 4),
        ("k_stride", ctypes.c_int64 * 4),
        ("v_stride", ctypes.c_int64 * 4),
        ("o_stride", ctypes.c_int64 * 4),
        ("sm_scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


SIGNATURES = {
    "rsfa_attention_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.c_void_p]),
    "rsfa_attention_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.c_void_p]),
    "rsfa_split_workspace_bytes": (ctypes.c_uint64, [_I64, _I64, _I64, _I64, _I32]),
    "rsfa_v8_workspace_bytes": (ctypes.c_uint64, [_I64, _I64, _I64, _I64]),
    "rsfa_get_tiling": (ctypes.c_int, [_I64, _I64, _I64, _I64, _I32, _I32, _PI32, _PI32]),
    "rsfa_resolve_tiling": (ctypes.c_int, [_I64, _I32, _I32, _I32, _I32, _PI32, _PI32]),
    "rsfa_get_num_compute_cores": (ctypes.c_int, [ctypes.c_int]),
    "rsfa_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "rsfa_abi_version": (ctypes.c_int, []),
}

_lib = None
_lock = threading.Lock()


def library_path():
    return _LIB_PATH


def lib():
    """The loaded librsfa.so (raises RuntimeError if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"ascend_rsfa native library not found at {_LIB_PATH}; build it with "
                    "`python ascend-rsfa_amd/build_native.py` (or __graft_entry__.build())")
            handle = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.rsfa_abi_version() != ABI_VERSION:
                raise RuntimeError("librsfa.so ABI version mismatch; rebuild the library")
            _lib = handle
    return _lib


def strerror(status):
    return lib().rsfa_strerror(status).decode()
