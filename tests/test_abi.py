"""C ABI checks that need no GPU: the library loads, exports every symbol the
header declares, rejects bad arguments with the documented codes before
touching a device, and its host-side repack implements the documented panel
layout."""
import ctypes
import os
import re

import numpy as np
import pytest

import madi_amd
from madi_amd import _lib, synth
import madi_amd.q8 as q8

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "madi_q8.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(madi_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = madi_amd.lib()
    syms = header_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    # and the ctypes binding declares exactly the header's API
    assert sorted(_lib.SIGNATURES) == syms


def test_header_compiles_as_c(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "madi_q8.h"\nint main(void){return MADI_OK;}\n')
    import subprocess
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    "-c", str(src), "-o", str(tmp_path / "t.o")], check=True)


FAKE = 0x100000  # 16-byte aligned, never dereferenced: every call below fails validation first

HANDLE_NAMES = ["dequant_q8_f16", "m4_gemm_nn", "m4_gemm_bias", "m4_gemm_bias_gelu", "gemv_q8",
                "gemv_q8_bias", "gemv_q8_bias_gelu", "gemv_q8_bias_res", "gemv_q8_qkv",
                "logit_gemv_q8", "gpu_emb_lookup_q8", "emb_lookup_indirect_q8", "emb_pe_rows_q8",
                "mul_mm_q8", "m4_flash_enc"]


def test_function_handles_by_name():
    """madi_get_function (mtl_get_function): one distinct handle per kernel name
    of the path, an error for any other name; the handle-taking wrappers
    refuse a handle of the wrong kind before touching a device."""
    ids = {name: q8.getFunction(name) for name in HANDLE_NAMES}
    assert len(set(ids.values())) == len(HANDLE_NAMES) and all(v > 0 for v in ids.values())
    out = ctypes.c_int(-1)
    assert madi_amd.lib().madi_get_function(b"layer_norm_f16", ctypes.byref(out)) == -9
    L = madi_amd.lib()
    assert L.madi_m4_gemm(ids["gemv_q8"], FAKE, FAKE, FAKE, None, 16, 256, 1280) == -9
    assert L.madi_q8_gemv_epi(ids["m4_gemm_bias"], FAKE, FAKE, FAKE, FAKE, FAKE, 256, 1280) == -9
    assert L.madi_m4_gemm(ids["m4_gemm_nn"], FAKE, FAKE, FAKE, None, 16, 256, 1280) == -8
    # the reference's two encoder attention kernels compute the same thing: one handle
    assert q8.getFunction("flash_attention_enc_f16") == ids["m4_flash_enc"]


@pytest.mark.parametrize("call,args,code", [
    ("madi_q8_gemm", (FAKE, FAKE, FAKE, FAKE, None, 0, 256, 1280, 0), -5),        # m == 0
    ("madi_q8_gemm", (FAKE, FAKE, FAKE, FAKE, None, 16, 100, 1280, 0), -5),       # n % 32
    ("madi_q8_gemm", (FAKE, FAKE, FAKE, FAKE, None, 16, 256, 96, 0), -5),         # k % 64
    ("madi_q8_gemm", (None, FAKE, FAKE, FAKE, None, 16, 256, 1280, 0), -6),       # null A
    ("madi_q8_gemm", (FAKE, FAKE, FAKE, FAKE, None, 16, 256, 1280, 1), -6),       # bias missing
    ("madi_q8_gemm", (FAKE, FAKE, FAKE, FAKE, FAKE, 16, 256, 1280, 3), -9),       # residual epi
    ("madi_q8_gemm", (FAKE + 2, FAKE, FAKE, FAKE, None, 16, 256, 1280, 0), -7),   # misaligned A
    ("madi_q8_gemm", (FAKE, FAKE, FAKE, FAKE, None, 16, 256, 1280, 0), -8),       # not initialised
    ("madi_q8_gemv", (FAKE, FAKE, FAKE, FAKE, 100, 96), -5),
    ("madi_q8_gemv", (FAKE, FAKE, FAKE + 8, FAKE, 100, 1280), -7),
    ("madi_q8_gemv", (FAKE, FAKE, FAKE, FAKE, 1 << 21, 1024), -5),                # 2 GiB weight
    ("madi_q8_emb_pe_rows", (FAKE, FAKE, FAKE, FAKE, FAKE, 96, 0, 4, 100), -5),   # dim % 64
    ("madi_q8_emb_pe_rows", (FAKE, FAKE, FAKE, None, FAKE, 1280, 0, 4, 100), -6), # null tokens
    ("madi_q8_emb_pe_rows", (FAKE, FAKE, FAKE, FAKE, FAKE + 4, 1280, 0, 4, 100), -7),  # pe
    ("madi_q8_emb_pe_rows", (FAKE, FAKE, FAKE, FAKE, FAKE, 1280, 0, 4, 100), -8),
    ("madi_q8_logit_gemv", (FAKE, FAKE, FAKE, FAKE, 1 << 22, 512), -5),           # 2 GiB vocab
    ("madi_q8_gemv", (FAKE, FAKE, FAKE, FAKE, 100, 1280), -8),
    ("madi_q8_gemv_bias", (FAKE, FAKE, FAKE, FAKE, None, 100, 1280), -6),
    ("madi_q8_gemv_qkv", (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 1280), -6),
    ("madi_q8_gemv_qkv", (FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1000), -5),
    ("madi_q8_gemv_f16x", (FAKE, FAKE, FAKE, FAKE, None, 100, 1280, 7), -9),
    ("madi_q8_logit_gemv", (FAKE, FAKE, FAKE, FAKE, 0, 1280), -5),
    ("madi_q8_dequant_f16", (FAKE, FAKE, FAKE, 1280, 1000), -5),
    ("madi_q8_dequant_f16", (FAKE, FAKE, FAKE, 1280, 1280), -8),
    ("madi_q8_repack", (FAKE, FAKE + 4096, FAKE, FAKE + 8192, 32, 64), -9),        # overlap
    ("madi_q8_emb_lookup", (FAKE, FAKE, FAKE, FAKE, 51866, 1000), -5),
    ("madi_q8_emb_lookup", (FAKE, FAKE, FAKE, None, 51866, 1280), -6),
    ("madi_q8_pproj", (FAKE, FAKE, FAKE, FAKE, 0, 1280, 1280), -5),               # m == 0
    ("madi_q8_pproj", (FAKE, FAKE, FAKE, FAKE, 65535 * 32 + 1, 32, 64), -5),      # slices > grid y
    ("madi_q8_pproj", (FAKE, None, FAKE, FAKE, 8, 1280, 1280), -6),
    ("madi_q8_pproj", (FAKE, FAKE + 4, FAKE, FAKE, 8, 1280, 1280), -7),
    ("madi_q8_pproj", (FAKE, FAKE, FAKE, FAKE, 65535 * 32, 32, 64), -8),         # largest M, not initialised
    ("madi_flash_enc_f16", (FAKE, FAKE + 0x10000, None, FAKE + 0x30000, 1500, 20), -6),
    ("madi_flash_enc_f16", (FAKE, FAKE + 0x1000000, FAKE + 0x2000000, FAKE + 0x3000000, 1500, 0), -5),
    ("madi_flash_enc_f16", (FAKE, FAKE, FAKE, FAKE, 1 << 21, 16), -5),            # > 2 GiB
    ("madi_flash_enc_f16", (FAKE, FAKE + 0x1000000, FAKE + 0x2000008, FAKE + 0x3000000, 1500, 20), -7),
    ("madi_flash_enc_f16", (FAKE, FAKE + 0x1000000, FAKE + 0x100000, FAKE + 0x3000000, 1500, 20), -9),  # out over k
    ("madi_flash_enc_f16", (FAKE, FAKE + 0x100, FAKE + 0x2000000, FAKE + 0x3000000, 1500, 20), -9),  # out over q
    ("madi_flash_enc_f16", (FAKE, FAKE, FAKE + 0x2000000, FAKE + 0x3000000, 1500, 20), -8),  # in place on q
    ("madi_q8_forget", (FAKE, 4096), -8),
    ("madi_matmul_f16", (FAKE, FAKE, FAKE, 0, 51866, 1280, 1.0, 0.0), -5),
    ("madi_matmul_f16", (FAKE, FAKE, FAKE, 8, 51866, 1280, 1.0, 0.0), -8),
    ("madi_alloc", (16,), None),
    ("madi_sync", (), -8),
    ("madi_upload", (FAKE, FAKE, 16), -8),
])
def test_error_codes_without_device(call, args, code):
    L = madi_amd.lib()
    rc = getattr(L, call)(*args)
    if code is None:  # madi_alloc returns NULL before init
        assert rc is None
        assert "madi_init" in _lib.last_error()
    else:
        assert rc == code, (_lib.last_error(), rc)
        assert _lib.last_error()


def test_madi_error_raised_by_wrappers():
    with pytest.raises(madi_amd.MadiError) as e:
        _lib.call("madi_q8_gemv", FAKE, FAKE, FAKE, FAKE, 100, 96)
    assert e.value.code == -5


# ------------------------------------------------------------------ panel layout spec
def layout_reference(qs, sc):
    """Direct transcription of the layout comment in include/madi_q8.h."""
    n, k = qs.shape
    tq = np.zeros(n * k, np.uint8)
    ts = np.zeros(n * (k // 32), np.float16)
    for p in range((n + 31) // 32):
        R = min(32, n - 32 * p)
        for c in range(k // 64):
            base = 32 * p * k + c * R * 64
            sbase = 32 * p * (k // 32) + c * 2 * R
            for j in range(2):
                for h in range(2):
                    for r in range(R):
                        off = base + ((2 * j + h) * R + r) * 16
                        src = qs[32 * p + r, 64 * c + 32 * h + 16 * j: 64 * c + 32 * h + 16 * j + 16]
                        tq[off:off + 16] = (src.astype(np.int16) + 128).astype(np.uint8)
            for h in range(2):
                for r in range(R):
                    ts[sbase + h * R + r] = sc[32 * p + r, 2 * c + h]
    return tq, ts


@pytest.mark.parametrize("n,k", [(32, 64), (70, 128), (96, 192)])
def test_host_repack_follows_documented_layout(n, k):
    rng = np.random.default_rng(n * k)
    qs, sc = synth.q8_weight(rng, n, k)
    tq, ts = q8.repack_host(qs, sc)
    rq, rs = layout_reference(qs, sc)
    assert np.array_equal(tq, rq)
    assert np.array_equal(ts.view(np.uint16), rs.view(np.uint16))


@pytest.mark.parametrize("n,k", [(1, 64), (31, 64), (33, 1280), (51866, 1280), (1280, 5120)])
def test_host_repack_round_trip(n, k):
    rng = np.random.default_rng(k)
    qs, sc = synth.q8_weight(rng, n, k)
    qs[0, :3] = [-128, -127, 127]  # the full int8 range survives the +128 bias
    tq, ts = q8.repack_host(qs, sc)
    q2, s2 = q8.unpack_host(tq, ts, n, k)
    assert np.array_equal(q2, qs)
    assert np.array_equal(s2.view(np.uint16), sc.view(np.uint16))


def test_panel_offsets_keep_row_slicing():
    """Repacking rows [32a, 32b) alone gives the same bytes as the slice of the
    whole repacked weight at the natural offsets (stacked q|k|v slicing)."""
    n, k = 3 * 96, 128
    rng = np.random.default_rng(4)
    qs, sc = synth.q8_weight(rng, n, k)
    tq, ts = q8.repack_host(qs, sc)
    for r0, r1 in [(0, 96), (96, 192), (192, 288), (32, 64)]:
        sq, ss = q8.repack_host(qs[r0:r1], sc[r0:r1])
        assert np.array_equal(tq[r0 * k:r1 * k], sq)
        assert np.array_equal(ts[r0 * (k // 32):r1 * (k // 32)].view(np.uint16), ss.view(np.uint16))
