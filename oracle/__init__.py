"""ctypes front-end of the CPU oracle (oracle/q8_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the madi_amd package.  Every function
takes and returns numpy arrays in the reference's natural Q8_0 layout
(qs int8 [N][K], scales float16 [N][K/32]).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libq8_oracle.so")

EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RES = 0, 1, 2, 3

_lib = None


def build() -> str:
    """Compile the oracle library with oracle/Makefile; returns its path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


NATIVE_FLAGS = ["-O3", "-march=native", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
                "-fPIC", "-shared"]


def build_native(out_dir: str) -> str | None:
    """Compile q8_oracle.c for the host it runs on (-march=native, the same
    -ffp-contract=off arithmetic) into out_dir; returns the library path, or
    None when no C compiler is available."""
    out = os.path.join(out_dir, "libq8_oracle_native.so")
    cc = os.environ.get("CC", "gcc")
    r = subprocess.run([cc, *NATIVE_FLAGS, "-o", out, os.path.join(_HERE, "q8_oracle.c"), "-lm"],
                       capture_output=True, text=True)
    return out if r.returncode == 0 and os.path.exists(out) else None


def use_library(path: str) -> None:
    """Load the oracle functions from another build of q8_oracle.c (e.g. the
    -march=native build of build_native)."""
    global _lib
    L = ctypes.CDLL(path)
    _declare(L)
    _lib = L


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_I = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    sig = {
        "oracle_f16_to_f32_array": (None, [_P, _P, ctypes.c_size_t]),
        "oracle_f32_to_f16_array": (None, [_P, _P, ctypes.c_size_t]),
        "oracle_gelu_erf": (ctypes.c_float, [ctypes.c_float]),
        "oracle_dequant_q8_f16": (None, [_P, _P, _P, _U32, _U32]),
        "oracle_q8_gemm_rows": (None, [_P, _P, _P, _P, _P, _I, _U32, _U32, _U32, _P, _U32, _I]),
        "oracle_q8_gemm_f16": (None, [_P, _P, _P, _P, _P, _I, _U32, _U32, _U32, _I]),
        "oracle_q8_gemv": (None, [_P, _P, _P, _P, _P, _I, _U32, _U32, _I]),
        "oracle_q8_gemv_qkv": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _U32, _U32]),
        "oracle_q8_proj": (None, [_P, _P, _P, _P, _U32, _U32, _U32, _I]),
        "oracle_quantize_q8": (None, [_P, _P, _P, _U32, _U32]),
        "oracle_fnv1a64": (ctypes.c_uint64, [ctypes.c_uint64, _P, ctypes.c_size_t]),
        "oracle_fnv_q8": (ctypes.c_uint64, [ctypes.c_uint64, _P, ctypes.c_size_t, _P, ctypes.c_size_t]),
        "oracle_emb_row_q8": (None, [_P, _P, _P, _U32, _U32]),
        "oracle_emb_pe_rows_q8": (None, [_P, _P, _P, _P, _P, _U32, _U32, _U32]),
        "oracle_gemm_f16": (None, [_P, _P, _P, _U32, _U32, _U32, ctypes.c_float, ctypes.c_float, _I]),
        "oracle_flash_enc_f16": (None, [_P, _P, _P, _P, _U32, _U32, _I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def _check_q8(qs, scales):
    n, k = qs.shape
    assert qs.dtype == np.int8 and k % 32 == 0
    assert scales.shape == (n, k // 32) and scales.dtype == np.float16
    return n, k


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_ptr(out), _ptr(h), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.float16)
    lib().oracle_f32_to_f16_array(_ptr(out), _ptr(f), f.size)
    return out


def gelu_erf(x: float) -> float:
    return lib().oracle_gelu_erf(x)


def dequant_q8_f16(qs, scales) -> np.ndarray:
    """f16 [K][N] (transposed), engine/metal/kernels/q8_gemm.metal:12-27."""
    n, k = _check_q8(qs, scales)
    qs, scales = _c(qs, np.int8), _c(scales, np.float16)
    out = np.empty((k, n), dtype=np.float16)
    lib().oracle_dequant_q8_f16(_ptr(out), _ptr(qs), _ptr(scales), n, k)
    return out


def q8_gemm_rows(a, qs, scales, rows=None, bias=None, epilogue=EPI_NONE, threads=1):
    """f32 results (epilogue applied) of A . deq(W)^T for the given row indices."""
    n, k = _check_q8(qs, scales)
    a = _c(a, np.float16)
    m = a.shape[0]
    assert a.shape == (m, k)
    qs, scales, bias = _c(qs, np.int8), _c(scales, np.float16), _c(bias, np.float32)
    if rows is None:
        out = np.empty((m, n), dtype=np.float32)
        lib().oracle_q8_gemm_rows(_ptr(out), _ptr(a), _ptr(qs), _ptr(scales), _ptr(bias),
                                  epilogue, m, n, k, None, 0, threads)
        return out
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    assert rows.size == 0 or int(rows.max()) < m
    out = np.empty((rows.size, n), dtype=np.float32)
    lib().oracle_q8_gemm_rows(_ptr(out), _ptr(a), _ptr(qs), _ptr(scales), _ptr(bias),
                              epilogue, m, n, k, _ptr(rows), rows.size, threads)
    return out


def q8_gemm_f16(a, qs, scales, bias=None, epilogue=EPI_NONE, threads=1):
    n, k = _check_q8(qs, scales)
    a = _c(a, np.float16)
    m = a.shape[0]
    qs, scales, bias = _c(qs, np.int8), _c(scales, np.float16), _c(bias, np.float32)
    out = np.empty((m, n), dtype=np.float16)
    lib().oracle_q8_gemm_f16(_ptr(out), _ptr(a), _ptr(qs), _ptr(scales), _ptr(bias),
                             epilogue, m, n, k, threads)
    return out


def q8_gemv(x, qs, scales, bias=None, epilogue=EPI_NONE, out=None, threads=1):
    n, k = _check_q8(qs, scales)
    x = _c(x, np.float32)
    assert x.shape == (k,)
    qs, scales, bias = _c(qs, np.int8), _c(scales, np.float16), _c(bias, np.float32)
    res = np.zeros(n, dtype=np.float32) if out is None else np.array(out, dtype=np.float32)
    lib().oracle_q8_gemv(_ptr(res), _ptr(x), _ptr(qs), _ptr(scales), _ptr(bias), epilogue,
                         n, k, threads)
    return res


def q8_gemv_qkv(x, qs, scales, qb, vb, kc, vc, pos):
    n, d = _check_q8(qs, scales)
    assert n == 3 * d
    x, qs, scales = _c(x, np.float32), _c(qs, np.int8), _c(scales, np.float16)
    qb, vb = _c(qb, np.float32), _c(vb, np.float32)
    kc, vc = np.array(kc, dtype=np.float32), np.array(vc, dtype=np.float32)
    q = np.zeros(d, dtype=np.float32)
    lib().oracle_q8_gemv_qkv(_ptr(q), _ptr(x), _ptr(qs), _ptr(scales), _ptr(qb), _ptr(vb),
                             _ptr(kc), _ptr(vc), pos, d)
    return q, kc, vc


def q8_proj(x_rows, qs, scales, threads=1):
    n, k = _check_q8(qs, scales)
    x_rows = _c(x_rows, np.float32)
    m = x_rows.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().oracle_q8_proj(_ptr(out), _ptr(x_rows), _ptr(_c(qs, np.int8)),
                         _ptr(_c(scales, np.float16)), m, n, k, threads)
    return out


def quantize_q8(w_f16):
    w = _c(w_f16, np.float16)
    rows, dim = w.shape
    assert dim % 32 == 0
    qs = np.empty((rows, dim), dtype=np.int8)
    sc = np.empty((rows, dim // 32), dtype=np.float16)
    lib().oracle_quantize_q8(_ptr(qs), _ptr(sc), _ptr(w), rows, dim)
    return qs, sc


FNV_SEED = 0xCBF29CE484222325


def fnv1a64(data: bytes, seed: int = FNV_SEED) -> int:
    buf = np.frombuffer(data, dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    return lib().oracle_fnv1a64(seed, _ptr(buf), len(data))


def fnv_q8(qs, scales, seed: int = FNV_SEED) -> int:
    qs, scales = _c(qs, np.int8), _c(scales, np.float16)
    return lib().oracle_fnv_q8(seed, _ptr(qs), qs.size, _ptr(scales), scales.size)


def emb_row_q8(qs, scales, tok: int):
    n, dim = _check_q8(qs, scales)
    assert 0 <= tok < n
    out = np.empty(dim, dtype=np.float32)
    lib().oracle_emb_row_q8(_ptr(out), _ptr(_c(qs, np.int8)), _ptr(_c(scales, np.float16)),
                            tok, dim)
    return out


def emb_pe_rows_q8(qs, scales, tokens, pe, pos0: int):
    """emb_pe_rows_q8 (decoder_ops.metal:614-633): [M][dim] f32 rows of the
    natural-layout table at `tokens` plus rows pos0.. of `pe`."""
    n, dim = _check_q8(qs, scales)
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    pe = np.ascontiguousarray(pe, dtype=np.float32)
    m = tokens.size
    assert np.all(tokens < n) and pe.shape[1] == dim and pos0 + m <= pe.shape[0]
    out = np.empty((m, dim), dtype=np.float32)
    lib().oracle_emb_pe_rows_q8(_ptr(out), _ptr(_c(qs, np.int8)), _ptr(_c(scales, np.float16)),
                                _ptr(tokens), _ptr(pe), dim, pos0, m)
    return out


def gemm_f16(a, b, c=None, alpha=1.0, beta=0.0, threads=1):
    a, b = _c(a, np.float16), _c(b, np.float16)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    out = np.zeros((m, n), dtype=np.float16) if c is None else np.array(c, dtype=np.float16)
    lib().oracle_gemm_f16(_ptr(out), _ptr(a), _ptr(b), m, n, k, alpha, beta, threads)
    return out


def flash_enc_f16(q, k, v, nh: int, threads=1):
    """m4_flash_enc (m4_gemm.metal:268-407): bidirectional attention with head
    dim 64 over f16 [seq][nh*64] q, k, v; returns f16 [seq][nh*64]."""
    q, k, v = _c(q, np.float16), _c(k, np.float16), _c(v, np.float16)
    seq, width = q.shape
    assert width == 64 * nh and k.shape == q.shape and v.shape == q.shape and seq >= 1
    out = np.zeros((seq, width), dtype=np.float16)
    lib().oracle_flash_enc_f16(_ptr(out), _ptr(q), _ptr(k), _ptr(v), seq, nh, threads)
    return out
