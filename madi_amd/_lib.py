"""ctypes binding of libmadi_q8.so (the C ABI declared in include/madi_q8.h).

The HIP library is the only implementation: if it is not built, loading fails
loudly; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# MADI_Q8_LIB may point at another build of the same library (e.g. a tuning variant)
LIB_PATH = os.environ.get("MADI_Q8_LIB", os.path.join(HERE, "libmadi_q8.so"))

MADI_OK = 0
ERRORS = {
    -1: "MADI_ERR_INIT", -2: "MADI_ERR_ALLOC", -3: "MADI_ERR_DISPATCH", -4: "MADI_ERR_SYNC",
    -5: "MADI_ERR_SHAPE", -6: "MADI_ERR_NULL", -7: "MADI_ERR_ALIGN", -8: "MADI_ERR_NOT_INIT",
    -9: "MADI_ERR_ARG",
}
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RES = 0, 1, 2, 3

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_I = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); every symbol include/madi_q8.h declares
SIGNATURES = {
    "madi_init": (_I, []),
    "madi_cleanup": (None, []),
    "madi_alloc": (_P, [_SZ]),
    "madi_free": (None, [_P]),
    "madi_upload": (_I, [_P, _P, _SZ]),
    "madi_download": (_I, [_P, _P, _SZ]),
    "madi_begin_command_buffer": (_I, []),
    "madi_commit_command_buffer": (_I, []),
    "madi_sync": (_I, []),
    "madi_set_stream": (_I, [_P]),
    "madi_last_error": (ctypes.c_char_p, []),
    "madi_device_cu_count": (_I, []),
    "madi_q8_repack_host": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "madi_q8_unpack_host": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "madi_q8_repack": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "madi_q8_quantize": (_I, [_P, _P, _P, _U32, _U32]),
    "madi_q8_fnv": (ctypes.c_uint64, [ctypes.c_uint64, _P, _SZ, _P, _SZ]),
    "madi_q8_dequant_f16": (_I, [_P, _P, _P, _U32, _U32]),
    "madi_q8_gemm": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _I]),
    "madi_q8_gemm_noalloc": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _I]),
    "madi_q8_gemv": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "madi_q8_gemv_bias": (_I, [_P, _P, _P, _P, _P, _U32, _U32]),
    "madi_q8_gemv_bias_gelu": (_I, [_P, _P, _P, _P, _P, _U32, _U32]),
    "madi_q8_gemv_bias_res": (_I, [_P, _P, _P, _P, _P, _U32, _U32]),
    "madi_q8_gemv_qkv": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _U32]),
    "madi_q8_logit_gemv": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "madi_q8_gemv_f16x": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _I]),
    "madi_q8_pproj": (_I, [_P, _P, _P, _P, _U32, _U32, _U32]),
    "madi_get_function": (_I, [ctypes.c_char_p, ctypes.POINTER(_I)]),
    "madi_m4_gemm": (_I, [_I, _P, _P, _P, _P, _U32, _U32, _U32]),
    "madi_q8_gemv_epi": (_I, [_I, _P, _P, _P, _P, _P, _U32, _U32]),
    "madi_proj_f16w": (_I, [_P, _P, _P, _P, _U32, _U32, _U32]),
    "madi_q8_materialize": (_I, [_P]),
    "madi_q8_forget": (_I, [_P, _SZ]),
    "madi_set_deferred_dequant": (_I, [_I]),
    "madi_set_gemm_grouping": (_I, [_I]),
    "madi_f16_gemm": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _I]),
    "madi_matmul_f16": (_I, [_P, _P, _P, _I, _I, _I, ctypes.c_float, ctypes.c_float]),
    "madi_q8_emb_lookup": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "madi_q8_emb_lookup_indirect": (_I, [_P, _P, _P, _P, _P, _U32, _U32]),
    "madi_q8_emb_pe_rows": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "madi_flash_enc_f16": (_I, [_P, _P, _P, _P, _U32, _U32]),
}


class MadiError(RuntimeError):
    def __init__(self, code: int, what: str, msg: str):
        super().__init__(f"{what} -> {ERRORS.get(code, code)}: {msg}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Load libmadi_q8.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m madi_amd.build` "
                "(the Q8 path has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().madi_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != MADI_OK:
        raise MadiError(rc, what, last_error())


_FNS: dict = {}


def call(name: str, *args) -> None:
    """Call export `name` and raise MadiError on a nonzero code (the function
    objects are looked up once: this is on every launch's host path)."""
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(lib(), name)
    rc = fn(*args)
    if rc != MADI_OK:
        raise MadiError(rc, name, last_error())
