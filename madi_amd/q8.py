"""Python mirror of the engine's Q8 matmul operator wrappers, over the C ABI.

Names, argument order and meaning follow the Zig wrappers the engine calls
(engine/metal/encoder.zig:125-159, engine/metal/decoder.zig:155-181,
engine/metal/transcribe.zig:4369-4393); a failing call raises MadiError, the
counterpart of the wrappers' error{DispatchFailed, ...} returns
(engine/metal/metal_backend.zig:34-41).  Pointers may be torch tensors (their
device address is passed) or plain integers.  torch supplies device memory and
the stream; all arithmetic runs in libmadi_q8.so.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from ._lib import EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RES, EPI_NONE, MadiError, call, check, lib

D = 1280          # encoder.zig:12, decoder.zig:12
MLP = 5120        # encoder.zig:15
VOCAB = 51866     # decoder.zig:19
ENC_SEQ = 1500    # encoder.zig:16
NH = 20           # encoder.zig:13 (attention heads, head dim 64: encoder.zig:14)


def ptr(t) -> int | None:
    if t is None or isinstance(t, int):
        return t
    return t.data_ptr()


def init(stream=None) -> None:
    """madi_init (mtl_init) and order launches on `stream` (a torch stream, a raw
    hipStream_t int, or None for torch's current stream)."""
    call("madi_init")
    if stream is None:
        import torch
        stream = torch.cuda.current_stream().cuda_stream
    elif not isinstance(stream, int):
        stream = stream.cuda_stream
    call("madi_set_stream", stream)


def sync() -> None:
    call("madi_sync")


def getFunction(name: str) -> int:
    """mtl.getFunction (metal_backend.zig:61-65) for this path's kernel names:
    the handle the handle-taking wrappers below expect."""
    import ctypes
    out = ctypes.c_int(-1)
    check(lib().madi_get_function(name.encode(), ctypes.byref(out)), f"madi_get_function({name})")
    return out.value


def _fn(f) -> int:
    return getFunction(f) if isinstance(f, str) else int(f)


def materialize(wdq=None) -> None:
    """Write a deferred kDeq / deqW16 result into wdq now (None: every one), for
    a reader outside the library (e.g. a torch copy of wdq)."""
    call("madi_q8_materialize", ptr(wdq))


def forget(buf, nbytes: int | None = None) -> None:
    """Announce a write by code outside the library (a torch copy, another
    kernel) into [buf, buf + nbytes): records of deferred dequantisations
    that the write would invalidate are dropped or materialised first."""
    if nbytes is None:
        nbytes = buf.numel() * buf.element_size()
    call("madi_q8_forget", ptr(buf), nbytes)


def set_deferred_dequant(on: bool) -> None:
    call("madi_set_deferred_dequant", 1 if on else 0)


@dataclass
class Q8:
    """A panel-layout Q8 weight on the device: {qs, scales} as in
    engine/metal/encoder.zig:21 (Q8) and decoder.zig:22 (Q8w)."""
    qs: int
    scales: int
    _keep: tuple = ()

    def rows(self, row0: int, k: int) -> "Q8":
        """The weight starting at row `row0` (a multiple of 32), as the engine slices
        stacked q|k|v weights (encoder.zig:263-267)."""
        assert row0 % 32 == 0, "panel layout slices at multiples of 32 rows"
        return Q8(self.qs + row0 * k, self.scales + row0 * (k // 32) * 2, self._keep)


def repack_host(qs: np.ndarray, scales: np.ndarray):
    """Natural Q8 (int8 [N][K], f16 [N][K/32]) -> panel layout, on the host."""
    n, k = qs.shape
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    tq = np.empty(n * k, dtype=np.uint8)
    ts = np.empty(n * (k // 32), dtype=np.float16)
    check(lib().madi_q8_repack_host(tq.ctypes.data, ts.ctypes.data, qs.ctypes.data,
                                    scales.ctypes.data, n, k), "madi_q8_repack_host")
    return tq, ts


def unpack_host(tq: np.ndarray, ts: np.ndarray, n: int, k: int):
    qs = np.empty((n, k), dtype=np.int8)
    sc = np.empty((n, k // 32), dtype=np.float16)
    check(lib().madi_q8_unpack_host(qs.ctypes.data, sc.ctypes.data,
                                    np.ascontiguousarray(tq).ctypes.data,
                                    np.ascontiguousarray(ts).ctypes.data, n, k),
          "madi_q8_unpack_host")
    return qs, sc


def upload_q8(qs: np.ndarray, scales: np.ndarray, device="cuda") -> Q8:
    """Load-time path: repack on the host, then copy to HBM.  Keeps the torch
    buffers alive inside the returned Q8."""
    import torch
    tq, ts = repack_host(qs, scales)
    dq = torch.from_numpy(tq).to(device)
    ds = torch.from_numpy(ts.view(np.int16)).to(device)
    return Q8(dq.data_ptr(), ds.data_ptr(), (dq, ds))


class _MadiBuf:
    """A madi_alloc allocation, freed with madi_free when dropped."""

    def __init__(self, nbytes: int):
        self.p = lib().madi_alloc(nbytes)
        if not self.p:
            raise MadiError(-2, "madi_alloc", _last_error())

    def __del__(self):
        if getattr(self, "p", None):
            try:
                lib().madi_free(self.p)
            except Exception:
                pass
            self.p = None


def _last_error() -> str:
    from ._lib import last_error
    return last_error()


def upload_q8_alloc(qs: np.ndarray, scales: np.ndarray) -> Q8:
    """Load-time path as the engine's loader runs it: the weight in its own
    madi_alloc allocation (mtl.alloc), repacked on the host and uploaded
    (madi_upload).  A stacked q|k|v weight loaded this way is what the q|k|v
    grouping recognises."""
    tq, ts = repack_host(qs, scales)
    bq, bs = _MadiBuf(tq.nbytes), _MadiBuf(ts.nbytes)
    call("madi_upload", bq.p, tq.ctypes.data, tq.nbytes)
    call("madi_upload", bs.p, ts.ctypes.data, ts.nbytes)
    return Q8(bq.p, bs.p, (bq, bs))


def set_gemm_grouping(on: bool) -> None:
    call("madi_set_gemm_grouping", 1 if on else 0)


def upload_q8_device_repack(qs: np.ndarray, scales: np.ndarray, device="cuda") -> Q8:
    """Load-time path: copy the natural rows to HBM, repack there (madi_q8_repack)."""
    import torch
    n, k = qs.shape
    nq = torch.from_numpy(np.ascontiguousarray(qs).view(np.uint8)).to(device)
    ns = torch.from_numpy(np.ascontiguousarray(scales).view(np.int16)).to(device)
    dq = torch.empty_like(nq)
    ds = torch.empty_like(ns)
    call("madi_q8_repack", dq.data_ptr(), ds.data_ptr(), nq.data_ptr(), ns.data_ptr(), n, k)
    return Q8(dq.data_ptr(), ds.data_ptr(), (dq, ds, nq, ns))


def quantize(w16, n: int, k: int, device="cuda") -> Q8:
    """Load-time quantisation on the GPU (quantInto, transcribe.zig:309-326, then
    the repack): F16 [n][k] device tensor -> panel-layout Q8 on the device."""
    import torch
    dq = torch.empty(n * k, dtype=torch.uint8, device=device)
    ds = torch.empty(n * (k // 32), dtype=torch.int16, device=device)
    call("madi_q8_quantize", dq.data_ptr(), ds.data_ptr(), ptr(w16), n, k)
    return Q8(dq.data_ptr(), ds.data_ptr(), (dq, ds))


FNV_SEED = 0xcbf29ce484222325


def fnv(seed: int, qs: np.ndarray, scales: np.ndarray) -> int:
    """fnvQ8 (transcribe.zig:131-140) over a natural-layout Q8 weight in host
    memory: FNV-1a 64 over the qs bytes, then the scales' bytes."""
    qs = np.ascontiguousarray(qs)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    return int(lib().madi_q8_fnv(seed, qs.ctypes.data, qs.size, scales.ctypes.data, scales.size))


# ---- encoder.zig -----------------------------------------------------------
def kDeq(wdq, w: Q8, n: int, k: int) -> None:
    """encoder.zig:154-159: Q8 [N][K] -> F16 [K][N] (dequant_q8_f16).  Deferred:
    an F16 GEMM on wdq runs the fused Q8 kernel; materialize(wdq) before reading
    wdq outside the library."""
    call("madi_q8_dequant_f16", ptr(wdq), w.qs, w.scales, n, k)


def deqW16(wdq, w: Q8, n: int, k: int) -> None:
    """transcribe.zig:4387-4393: same operator as kDeq."""
    kDeq(wdq, w, n, k)


def kGemmQ8(a, w: Q8, c, m: int, n: int, k: int) -> None:
    """Fused kDeq + kM4 (encoder.zig:125-130, 154-159): C = A . deq(W)^T, f16."""
    call("madi_q8_gemm", ptr(a), w.qs, w.scales, ptr(c), None, m, n, k, EPI_NONE)


def kGemmQ8Bias(a, w: Q8, c, bias, m: int, n: int, k: int, gelu: bool = False) -> None:
    """Fused kDeq + kM4Bias (encoder.zig:131-136) with the m4_gemm_bias or
    m4_gemm_bias_gelu epilogue (m4_gemm.metal:60-115)."""
    call("madi_q8_gemm", ptr(a), w.qs, w.scales, ptr(c), ptr(bias), m, n, k,
         EPI_BIAS_GELU if gelu else EPI_BIAS)


def kM4(f, a, b, c, m: int, n: int, k: int) -> None:
    """encoder.zig:125-130: C = A . B, f16 [M][K] . [K][N], f = the m4_gemm_nn
    handle (or its name).  b is an F16 weight or the wdq a kDeq just recorded
    (then the fused Q8 GEMM runs)."""
    call("madi_m4_gemm", _fn(f), ptr(a), ptr(b), ptr(c), None, m, n, k)


def kM4Bias(f, a, b, c, bias, m: int, n: int, k: int) -> None:
    """encoder.zig:131-136, f = the m4_gemm_bias or m4_gemm_bias_gelu handle."""
    call("madi_m4_gemm", _fn(f), ptr(a), ptr(b), ptr(c), ptr(bias), m, n, k)


def kFlash(f, out, q, k, v, seq: int, nh: int = NH) -> None:
    """encoder.zig:138-152: self-attention of one window over its Q, K, V
    projections (f16 [seq][nh*64] each), f = the m4_flash_enc or
    flash_attention_enc_f16 handle (or name); both run the same kernel."""
    global _FLASH_IDS
    if _FLASH_IDS is None:
        _FLASH_IDS = (getFunction("m4_flash_enc"), getFunction("flash_attention_enc_f16"))
    fid = _fn(f)
    if fid not in _FLASH_IDS:
        raise MadiError(-9, "kFlash", f"handle {fid} is not an encoder attention kernel")
    call("madi_flash_enc_f16", ptr(out), ptr(q), ptr(k), ptr(v), seq, nh)


_FLASH_IDS = None


def matmulF16Batched(a, b, c, m: int, n: int, k: int, alpha: float = 1.0,
                     beta: float = 0.0) -> None:
    """metal_backend.zig:120 -> mtl_matmul_f16_enc (metal_backend.h:103)."""
    call("madi_matmul_f16", ptr(a), ptr(b), ptr(c), m, n, k, alpha, beta)


# ---- decoder.zig -----------------------------------------------------------
def kGemvQ8(out, x, w: Q8, n: int, k: int) -> None:
    """decoder.zig:155-160 (gemv_q8)."""
    call("madi_q8_gemv", ptr(out), ptr(x), w.qs, w.scales, n, k)


def kGemvQ8Bias(out, x, w: Q8, bias, n: int, k: int) -> None:
    """decoder.zig:162-167 (gemv_q8_bias)."""
    call("madi_q8_gemv_bias", ptr(out), ptr(x), w.qs, w.scales, ptr(bias), n, k)


def kGemvQ8BiasEpi(f, out, x, w: Q8, bias, n: int, k: int) -> None:
    """decoder.zig:176-181; f = the gemv_q8_bias_gelu or gemv_q8_bias_res handle
    (or its name)."""
    call("madi_q8_gemv_epi", _fn(f), ptr(out), ptr(x), w.qs, w.scales, ptr(bias), n, k)


def pproj(in_f32, w: Q8, out_f32, M: int, N: int, Kk: int) -> None:
    """decoder.zig:427-432 (pproj: kDeq + kCvt32 + matmulF16Batched + kCvt16)
    as one fused kernel.  in_f32 [M][Kk] -> out_f32 [M][N]."""
    call("madi_q8_pproj", ptr(out_f32), ptr(in_f32), w.qs, w.scales, M, N, Kk)


def proj(in16, in_f32, w16, out_f32, B: int, N: int, Kk: int) -> None:
    """decoder.zig:337-341 (proj: kCvt32 + matmulF16Batched + kCvt16 on the
    F16 copy w16 of a Q8 weight); in16 is the BScratch staging buffer.  A w16
    that deqW16 recorded runs the fused batched projection on the Q8 weight."""
    call("madi_proj_f16w", ptr(out_f32), ptr(in_f32), ptr(w16), ptr(in16), B, N, Kk)


def kQkv(q_out, x, w: Q8, qb, vb, kc, vc, pos, d: int = D) -> None:
    """decoder.zig:169-174 (gemv_q8_qkv); pos is a device u32."""
    call("madi_q8_gemv_qkv", ptr(q_out), ptr(x), w.qs, w.scales, ptr(qb), ptr(vb), ptr(kc),
         ptr(vc), ptr(pos), d)


# ---- transcribe.zig ----------------------------------------------------------
def kLogitGemv(logits, qs: int, sc: int, x, vocab: int = VOCAB, dim: int = D) -> None:
    """transcribe.zig:4369-4374 (logit_gemv_q8)."""
    call("madi_q8_logit_gemv", ptr(logits), qs, sc, ptr(x), vocab, dim)


def embLookup(out, qs: int, sc: int, tok, vocab: int = VOCAB, dim: int = D) -> None:
    """transcribe.zig:4361-4366 (gpu_emb_lookup_q8), tok a device u32."""
    call("madi_q8_emb_lookup", ptr(out), qs, sc, ptr(tok), vocab, dim)


def embLookupIndirect(out, qs: int, sc: int, tokens, pos, vocab: int = VOCAB,
                      dim: int = D) -> None:
    """emb_lookup_indirect_q8 (graph_helpers.metal:354-367)."""
    call("madi_q8_emb_lookup_indirect", ptr(out), qs, sc, ptr(tokens), ptr(pos), vocab, dim)


def prefillEmbed(out, qs: int, sc: int, tokens, pe, pos0: int, M: int, dim: int = D,
                 vocab: int = VOCAB) -> None:
    """decoder.zig:460-467 (emb_pe_rows_q8): out[m] = emb(tokens[m]) + pe[pos0 + m]
    over the tied Q8 tok_emb; tokens a device u32 [M], pe a device f32 table."""
    call("madi_q8_emb_pe_rows", ptr(out), qs, sc, ptr(tokens), ptr(pe), dim, pos0, M, vocab)


def gemv_f16x(out, x16, w: Q8, n: int, k: int, bias=None, epilogue: int = EPI_NONE) -> None:
    """Q8 GEMV with fp16 activations (the measured decoder-GEMV configuration)."""
    call("madi_q8_gemv_f16x", ptr(out), ptr(x16), w.qs, w.scales, ptr(bias), n, k, epilogue)


__all__ = [
    "D", "MLP", "VOCAB", "ENC_SEQ", "NH", "Q8", "init", "sync", "getFunction", "materialize",
    "set_deferred_dequant", "forget", "repack_host", "unpack_host",
    "upload_q8", "upload_q8_alloc", "set_gemm_grouping", "upload_q8_device_repack", "quantize", "fnv", "FNV_SEED", "kDeq", "deqW16", "kGemmQ8", "kGemmQ8Bias", "kM4", "kM4Bias", "kFlash", "matmulF16Batched",
    "kGemvQ8", "kGemvQ8Bias", "kGemvQ8BiasEpi", "pproj", "proj", "kQkv", "kLogitGemv", "embLookup",
    "embLookupIndirect", "prefillEmbed", "gemv_f16x", "EPI_NONE", "EPI_BIAS", "EPI_BIAS_GELU",
    "EPI_BIAS_RES",
]
