"""A call list replayed from compiled code (libmadi_issue.so, csrc/issue.c).

The engine issues its operator calls from Zig (the decode loop,
engine/metal/transcribe.zig:2783-2800; the encoder's layer loop,
engine/metal/encoder.zig:256-303).  To measure a call sequence at the rate
compiled code issues it, build an IssueList once -- the same calls as the
Python wrappers in madi_amd.q8, recorded instead of made -- and run it: the C
loop makes the library calls, no Python between them.
"""
from __future__ import annotations

import ctypes
import os

from . import _lib
from .q8 import Q8, _fn, ptr

_HERE = os.path.dirname(os.path.abspath(__file__))
ISSUE_LIB = os.path.join(_HERE, "libmadi_issue.so")

GEMV, GEMV_BIAS, GEMV_EPI, QKV, LOGIT, PPROJ, DEQ, M4, Q8_GEMM, MATMUL_F16, FLASH = range(11)


class _Op(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("pad", ctypes.c_int32), ("a", ctypes.c_uint64 * 10)]


_issue = None


def lib() -> ctypes.CDLL:
    global _issue
    if _issue is None:
        _lib.lib()  # the library it calls, loaded first (same file)
        if not os.path.exists(ISSUE_LIB):
            raise RuntimeError(f"{ISSUE_LIB} is not built: run `python -m madi_amd.build`")
        L = ctypes.CDLL(ISSUE_LIB)
        L.madi_issue_run.restype = ctypes.c_int
        L.madi_issue_run.argtypes = [ctypes.POINTER(_Op), ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int64)]
        _issue = L
    return _issue


def _u(v) -> int:
    v = ptr(v)
    return 0 if v is None else int(v)


class IssueList:
    """Library calls recorded in order; run(reps) issues them reps times from C."""

    def __init__(self):
        self.ops: list[tuple[int, list[int]]] = []
        self._arr = None

    def _add(self, op, *args):
        self.ops.append((op, [_u(a) for a in args]))
        self._arr = None

    # the wrappers of madi_amd.q8, same argument order
    def kGemvQ8(self, out, x, w: Q8, n, k):
        self._add(GEMV, out, x, w.qs, w.scales, n, k)

    def kGemvQ8Bias(self, out, x, w: Q8, bias, n, k):
        self._add(GEMV_BIAS, out, x, w.qs, w.scales, bias, n, k)

    def kGemvQ8BiasEpi(self, f, out, x, w: Q8, bias, n, k):
        self._add(GEMV_EPI, _fn(f), out, x, w.qs, w.scales, bias, n, k)

    def kQkv(self, q_out, x, w: Q8, qb, vb, kc, vc, pos, d):
        self._add(QKV, q_out, x, w.qs, w.scales, qb, vb, kc, vc, pos, d)

    def kLogitGemv(self, logits, qs, sc, x, vocab, dim):
        self._add(LOGIT, logits, qs, sc, x, vocab, dim)

    def pproj(self, in_f32, w: Q8, out_f32, m, n, k):
        self._add(PPROJ, out_f32, in_f32, w.qs, w.scales, m, n, k)

    def kDeq(self, wdq, w: Q8, n, k):
        self._add(DEQ, wdq, w.qs, w.scales, n, k)

    def kM4(self, f, a, b, c, m, n, k):
        self._add(M4, _fn(f), a, b, c, 0, m, n, k)

    def kM4Bias(self, f, a, b, c, bias, m, n, k):
        self._add(M4, _fn(f), a, b, c, bias, m, n, k)

    def kGemmQ8(self, a, w: Q8, c, m, n, k, bias=None, epilogue=_lib.EPI_NONE):
        self._add(Q8_GEMM, a, w.qs, w.scales, c, bias, m, n, k, epilogue)

    def matmulF16Batched(self, a, b, c, m, n, k):
        self._add(MATMUL_F16, a, b, c, m, n, k)

    def kFlash(self, out, q, k, v, seq, nh):
        self._add(FLASH, out, q, k, v, seq, nh)

    def __len__(self):
        return len(self.ops)

    def run(self, reps: int = 1) -> None:
        if self._arr is None:
            arr = (_Op * max(len(self.ops), 1))()
            for i, (op, args) in enumerate(self.ops):
                arr[i].op = op
                for j, v in enumerate(args):
                    arr[i].a[j] = v
            self._arr = arr
        bad = ctypes.c_int64(-1)
        rc = lib().madi_issue_run(self._arr, len(self.ops), reps, ctypes.byref(bad))
        if rc != 0:
            op = self.ops[bad.value % len(self.ops)][0] if bad.value >= 0 else -1
            raise _lib.MadiError(rc, f"issue list call {bad.value} (op {op})", _lib.last_error())
