"""GPU parity of the gfx950 Q8 matmul path against the CPU oracle.

Every call goes through the C ABI (libmadi_q8.so via ctypes); torch only
provides device buffers.  Bars: bit-exact for the dequantised weights and the
layout work; normwise max|C - C_ref| / max|C_ref| <= 1e-3 (the path's
tolerance) for the GEMM/GEMV, where C_ref is the oracle's
dequantise-then-fp32-accumulate result.
"""
import sys

import numpy as np
import pytest

import oracle as O
from madi_amd import synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def q():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import madi_amd.q8 as q8
    q8.init()
    return q8


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16).view(np.int16)).cuda()


def host_f16(t):
    return t.cpu().numpy().view(np.float16)


def tight_ok(c, a, qs, sc):
    """Element-wise: the kernel must equal sum_k a_k * fp16_rne(q_k s_k) up to fp32
    accumulation (K * 2^-24 * sum|a||w16|) and one f16 output rounding
    (2^-11 relative, 2^-25 absolute below the normal range).  w16 comes from the
    oracle's bit-exact dequant; a wrong index or a dropped block breaks this by
    orders of magnitude."""
    w16 = O.dequant_q8_f16(qs, sc).astype(np.float64).T  # [N][K]
    a64 = a.astype(np.float64)
    exact = a64 @ w16.T
    bound = (2.0**-11 * np.abs(exact) + a.shape[1] * 2.0**-24 * (np.abs(a64) @ np.abs(w16).T)
             + 2.0**-25)
    return bool(np.all(np.abs(c.astype(np.float64) - exact) <= bound * 1.001))


def gelu_as64(v):
    """The erf-form GELU with the Abramowitz & Stegun 7.1.26 erf
    (graph_helpers.metal:460-473), evaluated in float64."""
    z = v / np.sqrt(2.0)
    az = np.abs(z)
    t = 1.0 / (1.0 + 0.3275911 * az)
    poly = t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027
                                                                           + t * 1.061405429))))
    erf = np.sign(z) * (1.0 - poly * np.exp(-az * az))
    return 0.5 * v * (1.0 + erf)


def tight_epi_ok(c, a, qs, sc, bias, gelu):
    """Element-wise for the bias / bias+GELU epilogues: the kernel must equal
    epi(sum_k a_k * fp16_rne(q_k s_k) + bias) up to fp32 accumulation (scaled
    by GELU's largest slope, 1.13), the GELU formula's fp32 evaluation (a few
    ulps) and one f16 output rounding."""
    w16 = O.dequant_q8_f16(qs, sc).astype(np.float64).T  # [N][K]
    a64 = a.astype(np.float64)
    v = a64 @ w16.T + bias.astype(np.float64)[None, :]
    acc = a.shape[1] * 2.0**-24 * (np.abs(a64) @ np.abs(w16).T) + 2.0**-24 * np.abs(v)
    exact, slope = (gelu_as64(v), 1.13) if gelu else (v, 1.0)
    bound = (2.0**-11 * np.abs(exact) + slope * acc + (4e-7 * (1.0 + np.abs(v)) if gelu else 0)
             + 2.0**-25)
    return bool(np.all(np.abs(c.astype(np.float64) - exact) <= bound * 1.001))


def normwise(c, ref):
    c = c.astype(np.float64)
    ref = ref.astype(np.float64)
    return np.max(np.abs(c - ref)) / max(np.max(np.abs(ref)), 1e-30)


def tile_rows(m):
    """Rows at every 32-row boundary of an m-row GEMM and a random sample."""
    edges = np.arange(0, m, 32)
    rows = np.r_[edges, edges - 1, m - 1, np.random.default_rng(m).integers(0, m, 8)]
    return np.unique(rows[(rows >= 0) & (rows < m)])


# ------------------------------------------------------------------ layout
@pytest.mark.parametrize("n,k", [(64, 128), (100, 256), (96, 320), (33, 192), (51866, 1280)])
def test_device_repack_matches_host(q, n, k):
    say(f"repack n={n} k={k}")
    rng = np.random.default_rng(n)
    qs, sc = synth.q8_weight(rng, n, k)
    tq, ts = q.repack_host(qs, sc)
    w = q.upload_q8_device_repack(qs, sc)
    q.sync()
    dq, ds = w._keep[0], w._keep[1]
    assert np.array_equal(dq.cpu().numpy().reshape(-1), tq)
    assert np.array_equal(ds.cpu().numpy().reshape(-1).view(np.uint16), ts.view(np.uint16))


@pytest.mark.parametrize("n,k", [(96, 128), (100, 256), (5120, 1280), (1280, 5120)])
def test_dequant_bit_exact(q, n, k):
    say(f"dequant n={n} k={k}")
    rng = np.random.default_rng(k + n)
    qs, sc = synth.q8_weight(rng, n, k)
    # subnormal and large scales too: bit-exactness must not depend on the range
    sc.flat[:8] = np.array([2**-24, 3 * 2**-24, 2**-14, 1e-5, 0.5, 1.0, 7.5, 300.0], np.float16)
    w = q.upload_q8(qs, sc)
    out = torch.empty((k, n), dtype=torch.int16, device="cuda")
    q.kDeq(out, w, n, k)
    q.materialize(out)  # torch reads wdq: the deferred dequantisation runs now
    q.sync()
    ref = O.dequant_q8_f16(qs, sc)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


def test_stacked_row_slices(q):
    """qkv slicing by pointer arithmetic (encoder.zig:263-267) on the panel layout."""
    d = 256
    rng = np.random.default_rng(3)
    qs, sc = synth.q8_weight(rng, 3 * d, d)
    w = q.upload_q8(qs, sc)
    for blk in range(3):
        out = torch.empty((d, d), dtype=torch.int16, device="cuda")
        q.kDeq(out, w.rows(blk * d, d), d, d)
        q.materialize(out)
        q.sync()
        ref = O.dequant_q8_f16(qs[blk * d:(blk + 1) * d], sc[blk * d:(blk + 1) * d])
        assert np.array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


# ------------------------------------------------------------------ GEMM
def _gemm(q, a, qs, sc, bias=None, gelu=False):
    m, k = a.shape
    n = qs.shape[0]
    w = q.upload_q8(qs, sc)
    da = dev_f16(a)
    dc = torch.empty((m, n), dtype=torch.int16, device="cuda")
    if bias is None:
        q.kGemmQ8(da, w, dc, m, n, k)
    else:
        q.kGemmQ8Bias(da, w, dc, dev(bias), m, n, k, gelu=gelu)
    q.sync()
    return host_f16(dc)


@pytest.mark.parametrize("m,n,k", [
    (50, 64, 128),      # the reference's correctness shape (K rounded up to the 64-wide chunk)
    (1, 256, 64),
    (33, 512, 1280),
    (100, 320, 192),    # N not a multiple of the 256-wide tile
    (257, 1280, 1280),  # out-proj / per-head q,k,v shape, M tail
])
def test_gemm_parity_small(q, m, n, k):
    say(f"gemm m={m} n={n} k={k}")
    a, qs, sc = synth.gemm_case(m * 7 + n, m, n, k)
    c = _gemm(q, a, qs, sc)
    ref = O.q8_gemm_rows(a, qs, sc, threads=8)
    assert normwise(c, ref) <= TOL, normwise(c, ref)
    assert tight_ok(c, a, qs, sc)


# One shape per m-tile height on a 256-CU device: 32-row tiles (m = 20, and
# m = 130, where 32-row tiles still fit one workgroup per CU), 64-row tiles
# (m = 33), 96-row tiles (m = 700 at n = 8192: 256 tiles, where 64-row tiles
# would be 352) and 128-row tiles (m = 800: 96-row tiles would be 288).
TILE_SHAPES = [(20, 320), (33, 320), (130, 320), (700, 8192), (800, 8192)]


@pytest.mark.parametrize("k", [128, 256, 320, 512, 768, 1024])
@pytest.mark.parametrize("m,n", TILE_SHAPES)
def test_gemm_k_loop_shapes(q, m, n, k):
    """Every K-loop shape at each m-tile height: chunk counts below eight or
    not a multiple of four run the padded loop (2, 4, 5 chunks); 8 chunks is
    one full trip plus the peeled last trip, 12 and 16 two and three trips."""
    say(f"gemm k-loop m={m} n={n} k={k}")
    a, qs, sc = synth.gemm_case(m * 13 + k, m, n, k)
    c = _gemm(q, a, qs, sc)
    rows = tile_rows(m)
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, threads=8)
    assert normwise(c[rows], ref) <= TOL, normwise(c[rows], ref)
    assert tight_ok(c[rows], a[rows], qs, sc)
    assert np.all(np.isfinite(c))


@pytest.mark.parametrize("m,n,k", [
    (257, 1280, 5120),  # 64-row tiles: 25 tiles x 4 K splits of 20 chunks, M tail
    (20, 512, 4096),    # 32-row tiles, 2 tiles x 4 splits of 16 chunks
    (64, 768, 6144),    # 64-row tiles, 3 tiles x 4 splits of 24 chunks
    (130, 512, 4288),   # 67 chunks: 4 splits of 16-17 chunks (padded loop)
    (1000, 1280, 5120),  # 80 tiles x 3 splits of 26-27 chunks (padded loop)
    (1100, 1280, 5120),  # 90 tiles x 2 splits of 40 chunks
])
def test_gemm_split_k(q, m, n, k):
    """Long K over few tiles: the workgroups of a tile split K and the last
    to finish adds the others' partial sums (run twice: the arrival counters
    must return to zero)."""
    say(f"gemm split-K m={m} n={n} k={k}")
    a, qs, sc = synth.gemm_case(m + n + k, m, n, k)
    ref = O.q8_gemm_rows(a, qs, sc, threads=8)
    for _ in range(2):
        c = _gemm(q, a, qs, sc)
        assert normwise(c, ref) <= TOL, normwise(c, ref)
        assert tight_ok(c, a, qs, sc)


@pytest.mark.parametrize("m,n,k,epi", [
    (1500, 1280, 6144, O.EPI_BIAS),       # 24 chunks per wave: four middle trips
    (1500, 1280, 4096, O.EPI_BIAS_GELU),  # 16 per wave (one middle trip), a 92-row last m-tile
    (1400, 1280, 5120, O.EPI_NONE),       # 20 per wave, 220 tiles, a 120-row last m-tile
    (1500, 1280, 5120, O.EPI_BIAS),       # fc2: 240 tiles
])
def test_gemm_ksplit_in_workgroup(q, m, n, k, epi):
    """Long K over few 128 x 256 tiles with N a multiple of 64: 128 x 64
    tiles whose four waves split K and meet in LDS (q8_gemm_ks_kernel).  Row
    sample over every 32-row boundary; a second run must give the same bits
    (the partials are added in wave order)."""
    say(f"gemm k-split in workgroup m={m} n={n} k={k} epi={epi}")
    a, qs, sc = synth.gemm_case(m + k, m, n, k)
    bias = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    b = None if epi == O.EPI_NONE else bias
    c = _gemm(q, a, qs, sc, bias=b, gelu=epi == O.EPI_BIAS_GELU)
    c2 = _gemm(q, a, qs, sc, bias=b, gelu=epi == O.EPI_BIAS_GELU)
    assert np.array_equal(c.view(np.uint16), c2.view(np.uint16))
    rows = tile_rows(m)
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=b, epilogue=epi, threads=16)
    assert normwise(c[rows], ref) <= TOL, normwise(c[rows], ref)
    if epi == O.EPI_NONE:
        assert tight_ok(c[rows], a[rows], qs, sc)
    else:
        assert tight_epi_ok(c[rows], a[rows], qs, sc, bias, epi == O.EPI_BIAS_GELU)
    assert np.all(np.isfinite(c))


def test_gemm_gelu_tails(q):
    """bias + GELU where the pre-activation spans +-40: the far negative tail
    must come out as (signed) zero and the positive tail as v itself, where
    e^(-z^2) underflows (fp32 exp2 below its range) and erf(|z|) is 1."""
    m, n, k = 33, 512, 128
    say(f"gemm gelu tails m={m} n={n} k={k}")
    a, qs, sc = synth.gemm_case(41, m, n, k)
    a = (a.astype(np.float32) * 0.01).astype(np.float16)
    bias = np.linspace(-40.0, 40.0, n).astype(np.float32)
    c = _gemm(q, a, qs, sc, bias=bias, gelu=True)
    assert np.all(np.isfinite(c))
    assert tight_epi_ok(c, a, qs, sc, bias, True)
    assert np.all(np.abs(c[:, :16].astype(np.float32)) < 1e-6)  # v < -37: GELU(v) ~ -1e-300


def test_gemm_one_hot_is_dequant(q):
    """A = identity rows: each output row is one dequantised weight column,
    bit-exact (one exact product, fp32 sum of zeros, exact f16 store)."""
    n, k = 256, 128
    rng = np.random.default_rng(5)
    qs, sc = synth.q8_weight(rng, n, k)
    a = np.eye(k, dtype=np.float16)
    c = _gemm(q, a, qs, sc)
    ref = O.dequant_q8_f16(qs, sc)  # [K][N]
    assert np.array_equal(c.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("m,n", TILE_SHAPES)
@pytest.mark.parametrize("gelu", [False, True])
def test_gemm_bias_epilogues(q, gelu, m, n):
    k = 640
    say(f"gemm bias gelu={gelu} m={m} n={n} k={k}")
    a, qs, sc = synth.gemm_case(11, m, n, k)
    bias = np.random.default_rng(12).standard_normal(n).astype(np.float32)
    c = _gemm(q, a, qs, sc, bias=bias, gelu=gelu)
    rows = tile_rows(m)
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=bias,
                         epilogue=O.EPI_BIAS_GELU if gelu else O.EPI_BIAS, threads=8)
    assert normwise(c[rows], ref) <= TOL
    assert tight_epi_ok(c[rows], a[rows], qs, sc, bias, gelu)
    assert np.all(np.isfinite(c))


# Every encoder and cross-attention projection at M = 1500 (one 30 s window)
# and the kernel instance it runs on a 256-CU device: fc1 128 x 256 tiles
# (240), q|k|v 96 x 256 tiles (240), cross K|V 128 x 128 tiles (240), out-proj
# 64 x 128 tiles (240), all with unpadded 20-chunk K loops; fc2 128 x 64 tiles
# (240) with K split four ways inside the workgroup (q8_gemm_ks_kernel, 20
# chunks per wave, the partials meeting in LDS).
ENCODER_SHAPES = [("fc1", 5120, 1280), ("fc2", 1280, 5120), ("qkv", 3840, 1280),
                  ("out", 1280, 1280), ("cross_kv", 2560, 1280)]


@pytest.mark.parametrize("name,n,k", ENCODER_SHAPES)
def test_gemm_encoder_shapes_full_m(q, name, n, k):
    """M = 1500; the oracle checks a row sample that covers every M-tile
    boundary and the tail, normwise and element-wise."""
    say(f"gemm encoder {name} m=1500 n={n} k={k}")
    m = 1500
    a, qs, sc = synth.gemm_case(0, m, n, k)
    c = _gemm(q, a, qs, sc)
    rows = np.unique(np.r_[tile_rows(m), 1, 129, 1498])  # every 32-row tile boundary
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, threads=16)
    assert normwise(c[rows], ref) <= TOL
    assert tight_ok(c[rows], a[rows], qs, sc)
    assert np.all(np.isfinite(c))


@pytest.mark.parametrize("name,n,k,gelu", [("fc1", 5120, 1280, True), ("fc2", 1280, 5120, False),
                                           ("qkv", 3840, 1280, False), ("out", 1280, 1280, False)])
def test_gemm_encoder_epilogues_full_m(q, name, n, k, gelu):
    """The encoder's production epilogue instances at M = 1500: fc1 + bias +
    GELU on 128 x 256 tiles with an unpadded 20-chunk loop, fc2 + bias where
    the four in-workgroup K ranges meet in LDS before the bias, q|k|v + bias
    on 96 x 256 and out + bias on 64 x 128 tiles (encoder.zig:262-301)."""
    say(f"gemm encoder epilogue {name} m=1500 n={n} k={k} gelu={gelu}")
    m = 1500
    a, qs, sc = synth.gemm_case(5, m, n, k)
    bias = np.random.default_rng(n + k).standard_normal(n).astype(np.float32)
    ref_rows = np.unique(np.r_[tile_rows(m), 1, 129, 1498])
    first = None
    for rep in range(2 if name == "fc2" else 1):  # split K: a rerun gives the same bits
        c = _gemm(q, a, qs, sc, bias=bias, gelu=gelu)
        if first is None:
            first = c.copy()
        assert np.array_equal(c.view(np.uint16), first.view(np.uint16)), rep
        ref = O.q8_gemm_rows(a, qs, sc, rows=ref_rows, bias=bias,
                             epilogue=O.EPI_BIAS_GELU if gelu else O.EPI_BIAS, threads=16)
        assert normwise(c[ref_rows], ref) <= TOL, rep
        assert tight_epi_ok(c[ref_rows], a[ref_rows], qs, sc, bias, gelu), rep
        assert np.all(np.isfinite(c))


@pytest.mark.parametrize("m,n,k,epi", [
    (33, 320, 512, O.EPI_NONE),         # 64-row tiles, one staging buffer, columns past N
    (60, 320, 768, O.EPI_BIAS_GELU),
    (700, 8000, 768, O.EPI_BIAS),       # 96-row tiles, columns past N, M tail
    (700, 8000, 1024, O.EPI_NONE),
    (800, 8000, 512, O.EPI_BIAS_GELU),  # 128-row tiles: one full trip, then the tail
    (1500, 5120, 1280, O.EPI_BIAS_GELU),  # fc1 of the encoder
    (1500, 2560, 1280, O.EPI_BIAS),     # cross K|V: 64-row tiles
])
def test_gemm_tail_matches_chunk_loop(q, m, n, k, epi):
    """The m-tile-major tail (the last four chunks one m-tile at a time, each
    m-tile's epilogue under the next one's MFMAs) against the chunk-by-chunk
    last trip (MADI_GEMM_TAIL=0): the accumulation order is the same, so the
    results agree bit for bit; the oracle checks a row sample of both."""
    import os
    say(f"gemm tail vs chunk loop m={m} n={n} k={k} epi={epi}")
    a, qs, sc = synth.gemm_case(m * 3 + n + k, m, n, k)
    bias = np.random.default_rng(k).standard_normal(n).astype(np.float32)
    b = None if epi == O.EPI_NONE else bias
    gelu = epi == O.EPI_BIAS_GELU
    old = os.environ.pop("MADI_GEMM_TAIL", None)
    try:
        c_tail = _gemm(q, a, qs, sc, bias=b, gelu=gelu)
        os.environ["MADI_GEMM_TAIL"] = "0"
        c_loop = _gemm(q, a, qs, sc, bias=b, gelu=gelu)
    finally:
        os.environ.pop("MADI_GEMM_TAIL", None)
        if old is not None:
            os.environ["MADI_GEMM_TAIL"] = old
    assert np.array_equal(c_tail.view(np.uint16), c_loop.view(np.uint16))
    rows = tile_rows(m)
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=b, epilogue=epi, threads=16)
    assert normwise(c_tail[rows], ref) <= TOL
    if b is None:
        assert tight_ok(c_tail[rows], a[rows], qs, sc)
    else:
        assert tight_epi_ok(c_tail[rows], a[rows], qs, sc, bias, gelu)
    assert np.all(np.isfinite(c_tail))


@pytest.mark.parametrize("m,n,k,epi", [
    (1500, 1280, 1280, O.EPI_NONE),       # out-proj: 64 x 128 tiles (24 x 10)
    (1500, 1280, 1280, O.EPI_BIAS_GELU),
    (1500, 2560, 1280, O.EPI_BIAS),       # cross K|V: 128 x 128 tiles (12 x 20)
    (1500, 2560, 1280, O.EPI_BIAS_GELU),
    (130, 320, 768, O.EPI_BIAS),          # a 2-row last m-tile, columns past N
    (200, 992, 512, O.EPI_NONE),          # 31 panels: the last tile has three
])
def test_gemm_narrow_tiles_match_wide(q, m, n, k, epi):
    """128-column tiles (one panel per wave, twice the rows) against the
    256-column tiles of the same shape (MADI_GEMM_NARROW=0): every output
    accumulates the same MFMAs in the same order, so the bits agree; the
    oracle checks a row sample, element-wise."""
    import os
    say(f"gemm narrow vs wide m={m} n={n} k={k} epi={epi}")
    a, qs, sc = synth.gemm_case(m + 5 * n + k, m, n, k)
    bias = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    b = None if epi == O.EPI_NONE else bias
    gelu = epi == O.EPI_BIAS_GELU
    old = os.environ.pop("MADI_GEMM_NARROW", None)
    try:
        c_narrow = _gemm(q, a, qs, sc, bias=b, gelu=gelu)
        os.environ["MADI_GEMM_NARROW"] = "0"
        c_wide = _gemm(q, a, qs, sc, bias=b, gelu=gelu)
    finally:
        os.environ.pop("MADI_GEMM_NARROW", None)
        if old is not None:
            os.environ["MADI_GEMM_NARROW"] = old
    assert np.array_equal(c_narrow.view(np.uint16), c_wide.view(np.uint16))
    rows = tile_rows(m)
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=b, epilogue=epi, threads=16)
    assert normwise(c_narrow[rows], ref) <= TOL
    if b is None:
        assert tight_ok(c_narrow[rows], a[rows], qs, sc)
    else:
        assert tight_epi_ok(c_narrow[rows], a[rows], qs, sc, bias, gelu)
    assert np.all(np.isfinite(c_narrow))


@pytest.mark.parametrize("name,n,k", [("fc1", 5120, 1280), ("fc2", 1280, 5120)])
def test_gemm_long_audio_full_m(q, name, n, k):
    """16 stacked windows, M = 24000: 128-row tiles, 188 x 20 (fc1) and 188 x 5
    (fc2) of them, several per CU; fc2's 80-chunk K runs unsplit and
    unpadded.  Row sample over tile boundaries, the tail and random rows."""
    say(f"gemm long audio {name} m=24000 n={n} k={k}")
    m = 24000
    rng = np.random.default_rng(24000 + n)
    a = synth.activations(rng, m, k)
    qs, sc = synth.q8_weight(rng, n, k)
    c = _gemm(q, a, qs, sc)
    rows = np.unique(np.r_[0, 31, 32, 127, 128, 255, 256, 12031, 12032, 23935, 23936,
                           23967, 23968, 23999, rng.integers(0, m, 24)])
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, threads=16)
    assert normwise(c[rows], ref) <= TOL
    assert tight_ok(c[rows], a[rows], qs, sc)
    assert np.all(np.isfinite(c))


@pytest.mark.parametrize("m,n,k,epi", [
    (24000, 5120, 1280, O.EPI_NONE),       # long-audio fc1: 3760 tiles, 14.7 per workgroup
    (24000, 5120, 1280, O.EPI_BIAS_GELU),  # ... with bias + GELU
    (7001, 4096, 768, O.EPI_BIAS_GELU),    # 12-chunk K (first trip, one middle, last), M tail of 89 rows
    (13300, 1280, 2048, O.EPI_BIAS),       # 520 tiles: two rounds and 8 tiles, 32-chunk K, M tail of 116
])
def test_gemm_persistent(q, m, n, k, epi):
    """At least two rounds of 128 x 256 tiles: the persistent tile loop
    (q8_gemm_persist_kernel) issues each next tile's loads before the
    finished tile's epilogue.  Row sample over tile boundaries and the tail;
    a second run gives the same bits."""
    say(f"gemm persistent m={m} n={n} k={k} epi={epi}")
    rng = np.random.default_rng(m + n)
    a = synth.activations(rng, m, k)
    qs, sc = synth.q8_weight(rng, n, k)
    bias = rng.standard_normal(n).astype(np.float32)
    b = None if epi == O.EPI_NONE else bias
    c = _gemm(q, a, qs, sc, bias=b, gelu=epi == O.EPI_BIAS_GELU)
    c2 = _gemm(q, a, qs, sc, bias=b, gelu=epi == O.EPI_BIAS_GELU)
    assert np.array_equal(c.view(np.uint16), c2.view(np.uint16))
    rows = np.unique(np.r_[0, 31, 32, 127, 128, 255, 256, (m // 128) * 128 - 1, (m // 128) * 128,
                           m // 2, m - 33, m - 1, rng.integers(0, m, 24)])
    rows = rows[(rows >= 0) & (rows < m)]
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=b, epilogue=epi, threads=16)
    assert normwise(c[rows], ref) <= TOL, normwise(c[rows], ref)
    if epi == O.EPI_NONE:
        assert tight_ok(c[rows], a[rows], qs, sc)
    else:
        assert tight_epi_ok(c[rows], a[rows], qs, sc, bias, epi == O.EPI_BIAS_GELU)
    assert np.all(np.isfinite(c))


def test_gemm_large_m(q):
    """Several tiles per CU (M = 6657: 53 x 20 tiles of 128 x 256, a 1-row M
    tail); row sample over tile boundaries."""
    m, n, k = 6657, 5120, 1280
    say(f"gemm large m={m} n={n} k={k}")
    a, qs, sc = synth.gemm_case(9, m, n, k)
    c = _gemm(q, a, qs, sc)
    rows = np.unique(np.r_[0, 31, 32, 255, 256, 257, 511, 512, 4095, 4096, 6400, 6655, 6656,
                           np.random.default_rng(2).integers(0, m, 12)])
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, threads=16)
    assert normwise(c[rows], ref) <= TOL
    assert tight_ok(c[rows], a[rows], qs, sc)
    assert np.all(np.isfinite(c))


# ------------------------------------------------------------------ GEMV
# (51866, 1280): four waves per panel; the others sixteen: (3840, 1280),
# (5120, 1280), (40, 64) one or two chunks per wave, (1280, 5120) four K
# splits, (5120, 4096) four chunks per wave through the two-chunk window,
# (40, 12288) the largest K in four splits of 48 chunks
# Shapes: the vocab and the decoder projections; 40 panels at K = 64 (one
# chunk: fifteen of the sixteen waves own none); 5120 x 4096 (four chunks per
# wave, past the first window); 40 x 12288 (K split over workgroups); and
# wide matrices (256 or more panels, four waves, the fp32 vector read one
# unit ahead) at K = 64 and 192, where some waves own no chunk and others one.
@pytest.mark.parametrize("n,k", [(51866, 1280), (3840, 1280), (1280, 5120), (5120, 1280), (40, 64),
                                 (5120, 4096), (40, 12288), (8200, 64), (8192, 192)])
def test_gemv_parity(q, n, k):
    say(f"gemv n={n} k={k}")
    x16, qs, sc = synth.gemv_case(n + k, n, k)
    x = x16.astype(np.float32)
    w = q.upload_q8(qs, sc)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    q.kGemvQ8(out, dev(x), w, n, k)
    q.sync()
    ref = O.q8_gemv(x, qs, sc, threads=8)
    got = out.cpu().numpy()
    assert normwise(got, ref) <= TOL
    # f32 accumulation both sides: far tighter than the gate in practice
    assert normwise(got, ref) <= 1e-5
    # the fp16-activation entry point computes the same sums
    out2 = torch.empty(n, dtype=torch.float32, device="cuda")
    q.gemv_f16x(out2, dev_f16(x16), w, n, k)
    q.sync()
    assert normwise(out2.cpu().numpy(), ref) <= 1e-5


@pytest.mark.parametrize("x_f16", [False, True])
def test_gemv_zero_blocks_are_exact(q, x_f16):
    """All-zero quantisation blocks (scale 1.0) contribute exactly nothing:
    a row of zero blocks gives exactly 0, and zero blocks mixed into a row
    leave its sum at the oracle's to f32 rounding."""
    n, k = 96, 1280
    x16, qs, sc = synth.gemv_case(71, n, k)
    qs[5, :] = 0
    sc[5, :] = 1.0
    qs[7, 64:256] = 0
    sc[7, 2:8] = 1.0
    w = q.upload_q8(qs, sc)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    if x_f16:
        q.gemv_f16x(out, dev_f16(x16), w, n, k)
    else:
        q.kGemvQ8(out, dev(x16.astype(np.float32)), w, n, k)
    q.sync()
    got = out.cpu().numpy()
    assert got[5] == 0.0
    ref = O.q8_gemv(x16.astype(np.float32), qs, sc, threads=4)
    assert normwise(got, ref) <= 1e-5


@pytest.mark.parametrize("case", ["full_mantissa", "huge", "tiny", "mixed_in_block", "zero_blocks"])
def test_gemv_f32_activations(q, case):
    """f32 activations with full 24-bit mantissas and wide ranges: the kernel
    multiplies each f32 x by the exact integer q in fp32 FMAs, one partial sum
    per 32-element block, then scales the partial by the block's scale.  Bar
    per row: the float64 sum within (K 2^-24 + 2^-21) sum_k |x_k q_k s_k|
    (fp32 accumulation), far below what a lost scale factor or a dropped
    block makes."""
    n, k = 256, 1280
    rng = np.random.default_rng(7 * len(case) + ord(case[0]))
    qs, sc = synth.q8_weight(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    if case == "huge":
        x *= np.float32(3e30)
    elif case == "tiny":
        x *= np.float32(2e-30)
    elif case == "mixed_in_block":
        x *= (10.0 ** rng.uniform(-6, 6, k)).astype(np.float32)
    elif case == "zero_blocks":
        x[64:160] = 0.0
        x[1000:1024] = 0.0
    say(f"gemv f32 x {case}")
    w = q.upload_q8(qs, sc)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    q.kGemvQ8(out, dev(x), w, n, k)
    q.sync()
    got = out.cpu().numpy().astype(np.float64)
    w64 = (qs.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=1))  # [N][K]
    exact = w64 @ x.astype(np.float64)
    mag = np.abs(w64) @ np.abs(x.astype(np.float64))
    bound = (k * 2.0**-24 + 2.0**-21) * mag
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - exact) <= bound), np.max(np.abs(got - exact) / np.maximum(bound, 1e-300))
    ref = O.q8_gemv(x, qs, sc, threads=4)
    assert normwise(got, ref) <= 1e-5


def test_logit_gemv_vocab(q):
    n, k = 51866, 1280
    x16, qs, sc = synth.gemv_case(0, n, k)
    x = x16.astype(np.float32)
    w = q.upload_q8(qs, sc)
    logits = torch.empty(n, dtype=torch.float32, device="cuda")
    q.kLogitGemv(logits, w.qs, w.scales, dev(x), n, k)
    q.sync()
    ref = O.q8_gemv(x, qs, sc, threads=8)
    got = logits.cpu().numpy()
    assert normwise(got, ref) <= 1e-5
    assert int(np.argmax(got)) == int(np.argmax(ref))


@pytest.mark.parametrize("n,k", [(5120, 1280), (1280, 5120)])  # the second splits K over workgroups
@pytest.mark.parametrize("epi", ["bias", "gemv_q8_bias_gelu", "gemv_q8_bias_res"])
def test_gemv_epilogues(q, epi, n, k):
    x16, qs, sc = synth.gemv_case(7, n, k)
    x = x16.astype(np.float32)
    rng = np.random.default_rng(8)
    bias = rng.standard_normal(n).astype(np.float32)
    res0 = rng.standard_normal(n).astype(np.float32)
    w = q.upload_q8(qs, sc)
    out = dev(res0.copy())
    if epi == "bias":
        q.kGemvQ8Bias(out, dev(x), w, dev(bias), n, k)
        ref = O.q8_gemv(x, qs, sc, bias, O.EPI_BIAS)
    elif epi == "gemv_q8_bias_gelu":
        q.kGemvQ8BiasEpi(epi, out, dev(x), w, dev(bias), n, k)
        ref = O.q8_gemv(x, qs, sc, bias, O.EPI_BIAS_GELU)
    else:
        q.kGemvQ8BiasEpi(epi, out, dev(x), w, dev(bias), n, k)
        ref = O.q8_gemv(x, qs, sc, bias, O.EPI_BIAS_RES, out=res0)
    q.sync()
    assert normwise(out.cpu().numpy(), ref) <= 1e-5


def test_gemv_qkv_kv_store(q):
    d = 1280
    x16, qs, sc = synth.gemv_case(9, 3 * d, d)
    x = x16.astype(np.float32)
    rng = np.random.default_rng(10)
    qb = rng.standard_normal(d).astype(np.float32)
    vb = rng.standard_normal(d).astype(np.float32)
    kc0 = np.full((8, d), 5.0, np.float32)
    vc0 = np.full((8, d), -5.0, np.float32)
    w = q.upload_q8(qs, sc)
    qo = torch.empty(d, dtype=torch.float32, device="cuda")
    kc, vc = dev(kc0.copy()), dev(vc0.copy())
    pos = torch.tensor([6], dtype=torch.int32, device="cuda")
    q.kQkv(qo, dev(x), w, dev(qb), dev(vb), kc, vc, pos, d)
    q.sync()
    rq, rk, rv = O.q8_gemv_qkv(x, qs, sc, qb, vb, kc0, vc0, 6)
    assert normwise(qo.cpu().numpy(), rq) <= 1e-5
    gk, gv = kc.cpu().numpy(), vc.cpu().numpy()
    assert normwise(gk[6], rk[6]) <= 1e-5 and normwise(gv[6], rv[6]) <= 1e-5
    others = np.r_[0:6, 7]
    assert np.all(gk[others] == 5.0) and np.all(gv[others] == -5.0)


def test_emb_lookup_rows(q):
    n, k = 51866, 1280
    rng = np.random.default_rng(21)
    qs, sc = synth.q8_weight(rng, n, k)
    w = q.upload_q8(qs, sc)
    out = torch.empty(k, dtype=torch.float32, device="cuda")
    for tok in (0, 31, 32, 50257, 51865):
        t = torch.tensor([tok], dtype=torch.int32, device="cuda")
        q.embLookup(out, w.qs, w.scales, t, n, k)
        q.sync()
        assert np.array_equal(out.cpu().numpy(), O.emb_row_q8(qs, sc, tok)), tok
    toks = torch.tensor([7, 51864, 3], dtype=torch.int32, device="cuda")
    pos = torch.tensor([1], dtype=torch.int32, device="cuda")
    q.embLookupIndirect(out, w.qs, w.scales, toks, pos, n, k)
    q.sync()
    assert np.array_equal(out.cpu().numpy(), O.emb_row_q8(qs, sc, 51864))


@pytest.mark.parametrize("m,pos0", [(1, 0), (4, 7), (37, 100), (320, 128)])
def test_emb_pe_rows(q, m, pos0):
    """Sequence prefill's embedding (emb_pe_rows_q8 behind prefillEmbed) from
    the panel-layout tied tok_emb, bit-exact against the oracle: tokens from
    every part of the vocab including the 26-row last panel; an
    out-of-vocab token leaves its row untouched."""
    n, k = 51866, 1280
    say(f"emb_pe_rows m={m} pos0={pos0}")
    rng = np.random.default_rng(m + pos0)
    qs, sc = synth.q8_weight(rng, n, k)
    w = q.upload_q8(qs, sc)
    toks = rng.integers(0, n, m).astype(np.uint32)
    toks[: min(m, 4)] = np.array([0, 51865, 51840, 31], np.uint32)[: min(m, 4)]
    pe = rng.standard_normal((448, k)).astype(np.float32)
    out = torch.full((m, k), 7.0, dtype=torch.float32, device="cuda")
    tt = toks.copy()
    if m > 4:
        tt[4] = n  # out of range: row stays at 7.0
    q.prefillEmbed(out, w.qs, w.scales, dev(tt.view(np.int32)), dev(pe), pos0, m, k, n)
    q.sync()
    got = out.cpu().numpy()
    ref = O.emb_pe_rows_q8(qs, sc, toks, pe, pos0)
    keep = np.ones(m, bool)
    if m > 4:
        keep[4] = False
        assert np.all(got[4] == 7.0)
    assert np.array_equal(got[keep], ref[keep])


# ------------------------------------------------------------------ batched / skinny projection
def _pproj(q, x, qs, sc):
    m, k = x.shape
    n = qs.shape[0]
    w = q.upload_q8(qs, sc)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    q.pproj(dev(x), w, out, m, n, k)
    q.sync()
    return out.cpu().numpy()


def staged_ok(c, x, qs, sc):
    """Element-wise: pproj must equal sum_k f16(x_k) * fp16_rne(q_k s_k) (the
    f16 staging of decoder.zig:427-432) up to fp32 accumulation error
    (K * 2^-24 * sum|x16||w16|); it stores f32, so no output rounding."""
    x16 = O.f32_to_f16(x).astype(np.float64)
    w16 = O.dequant_q8_f16(qs, sc).astype(np.float64)  # [K][N]
    exact = x16 @ w16
    bound = x.shape[1] * 2.0**-24 * (np.abs(x16) @ np.abs(w16)) + 2.0**-40
    return bool(np.all(np.abs(c.astype(np.float64) - exact) <= bound * 1.001))


@pytest.mark.parametrize("m,n,k", [
    (1, 3840, 1280), (2, 3840, 1280), (8, 5120, 1280), (16, 1280, 5120),
    (8, 51866, 1280),    # batched vocab logits, tail panel of 26 rows
    (24, 51866, 1280),   # vocab with 32-row slices: four panels per workgroup
    (3, 51866, 1280), (13, 51866, 1280),  # vocab, 8-row tiles (one panel per
                                          # workgroup) and 16-row tiles (four): rows past M
    (32, 1280, 1280), (33, 3840, 1280), (70, 1280, 5120), (5, 40, 64),
    (17, 5120, 1280),    # one 32-row slice, 15 rows past M
    (320, 640, 1280),    # ten slices (M = 320, the prefill's largest) of 20 panels
    (192, 1280, 1280),   # six slices of 40 panels: 240 workgroups, the most that
                         # stay on the skinny kernel for a 1280 x 1280 weight
    # the batched decode step at M = 16: vocab (four panels per workgroup, tail panel),
    # q|k|v, FFN up and the 1280 x 1280 projections (single panels, unsplit)
    (16, 51866, 1280), (16, 3840, 1280), (16, 5120, 1280), (16, 1280, 1280),
    # single panels, K unsplit (128 or more panels) and longer than one window
    # per wave: the staged first window, then the chunk-by-chunk loop
    (8, 5120, 4096), (3, 4096, 2048),
    # panel pairs (a workgroup per panel and slice would not fit the CUs):
    # the prefill's 1280 x 1280 at M = 320 and 224, an odd panel count (the
    # last pair holds one valid panel and a clamped one), and a partial last
    # panel with an M tail and a 10-chunk K
    (320, 1280, 1280), (224, 1280, 1280), (320, 1312, 1280), (300, 1000, 640),
])
def test_pproj_parity(q, m, n, k):
    say(f"pproj m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 131 + n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    qs, sc = synth.q8_weight(rng, n, k)
    c = _pproj(q, x, qs, sc)
    assert np.all(np.isfinite(c))
    ref = O.q8_proj(x, qs, sc, threads=8)   # test_batchproj.zig:72-78, f32 throughout
    assert normwise(c, ref) <= TOL, normwise(c, ref)
    assert staged_ok(c, x, qs, sc)


# From 160 rows, for weights 2048 wide or 4096 long, or where the skinny
# kernel's grid (panels x 32-row slices) exceeds the CUs, the batched
# projection runs as the MFMA GEMM with f32 activations and an f32 result
# (q8_gemm_kernel<MT, NONE, PADDED, true, false, PW>): 32 x 128, 64 x 128 and
# 64 x 256 tiles, an M tail, a padded K loop (5 chunks over 4096 outputs) and
# the 5120-wide K split over workgroups; 2048-wide weights at 224 and 288
# rows (32 x 128 tiles), and 1280 x 1280 at 600 rows, where even panel pairs
# would not fit the CUs.
@pytest.mark.parametrize("m,n,k", [
    (160, 5120, 1280), (320, 3840, 1280), (320, 5120, 1280), (161, 4096, 320),
    (320, 1280, 5120), (700, 2560, 1280), (224, 2048, 1280), (288, 2048, 1280),
    (600, 1280, 1280),
])
def test_pproj_many_rows_gemm(q, m, n, k):
    say(f"pproj (GEMM) m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 7 + n + k)
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    qs, sc = synth.q8_weight(rng, n, k)
    c = _pproj(q, x, qs, sc)
    assert np.all(np.isfinite(c))
    ref = O.q8_proj(x, qs, sc, threads=16)
    assert normwise(c, ref) <= TOL, normwise(c, ref)
    assert staged_ok(c, x, qs, sc)


# Where the batched projection would run 32-row tiles, or 64-row tiles with K
# split four ways over workgroups, and the K loop is unpadded, it runs
# 32 x 128 or 64 x 128 tiles (one panel per wave): the same MFMAs per output
# in the same order and the same splits summed in the same order, so the f32
# results equal the 256-column tiles' (MADI_GEMM_NARROW=0) bit for bit.
# Shapes: the prefill's q|k|v, FFN up and FFN down (four splits) at M = 320
# (64 x 128), cross K|V (32 x 128), 1280 x 1280 at M = 600 (32 x 128), FFN
# up at M = 160 (32 x 128), an M tail of 33 rows, 65 panels (the last tile
# holds one valid panel and three clamped ones), FFN down at M = 160 (a
# 32-row tail in a 64-row tile), a 2048-wide weight at M = 231 (a 7-row tail
# in a 32-row tile), and a 96-wide weight with K = 4096 (one tile of three
# panels and a clamped fourth, K split four ways).
@pytest.mark.parametrize("m,n,k", [
    (320, 3840, 1280), (320, 5120, 1280), (161, 2048, 512), (320, 2080, 1280),
    (320, 1280, 5120), (160, 1280, 5120), (600, 1280, 1280), (320, 2560, 1280),
    (160, 5120, 1280), (231, 2048, 1280), (300, 96, 4096),
])
def test_pproj_narrow_tiles_match_wide(q, m, n, k):
    import os
    say(f"pproj (GEMM) narrow vs wide m={m} n={n} k={k}")
    rng = np.random.default_rng(m * 11 + n + k)
    x = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    qs, sc = synth.q8_weight(rng, n, k)
    old = os.environ.pop("MADI_GEMM_NARROW", None)
    try:
        c_narrow = _pproj(q, x, qs, sc)
        os.environ["MADI_GEMM_NARROW"] = "0"
        c_wide = _pproj(q, x, qs, sc)
    finally:
        os.environ.pop("MADI_GEMM_NARROW", None)
        if old is not None:
            os.environ["MADI_GEMM_NARROW"] = old
    assert np.all(np.isfinite(c_narrow))
    assert np.array_equal(c_narrow.view(np.uint32), c_wide.view(np.uint32))
    ref = O.q8_proj(x, qs, sc, threads=16)
    assert normwise(c_narrow, ref) <= TOL, normwise(c_narrow, ref)
    assert staged_ok(c_narrow, x, qs, sc)


def test_pproj_many_rows_one_hot(q):
    """One-hot rows through the GEMM route: f32 results equal the dequantised
    weights bit for bit (one exact product, exact fp32 sums, f32 store)."""
    n, k = 2048, 256
    rng = np.random.default_rng(19)
    qs, sc = synth.q8_weight(rng, n, k)
    ks = np.arange(170) % k
    x = np.zeros((len(ks), k), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    c = _pproj(q, x, qs, sc)
    ref = O.dequant_q8_f16(qs, sc)[ks].astype(np.float32)
    assert np.array_equal(c, ref)


@pytest.mark.parametrize("n", [1280, 1312])
def test_pproj_panel_pairs_one_hot(q, n):
    """One-hot rows through the panel-pair route (256 rows of a 1280-long
    weight: a workgroup per panel and slice would not fit the CUs, a
    workgroup per pair does; 1312 = 41 panels leaves the last pair one valid
    panel): the f32 results equal the dequantised weights bit for bit."""
    k = 1280
    rng = np.random.default_rng(23)
    qs, sc = synth.q8_weight(rng, n, k)
    ks = (np.arange(256) * 37) % k
    x = np.zeros((len(ks), k), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    c = _pproj(q, x, qs, sc)
    ref = O.dequant_q8_f16(qs, sc)[ks].astype(np.float32)
    assert np.array_equal(c, ref)


@pytest.mark.parametrize("m", [8, 16])
def test_pproj_vocab_one_hot(q, m):
    """One-hot rows through the vocab's launch shapes (8 rows: one panel per
    workgroup; 16: four panels per workgroup, the last group ending in the
    26-row tail panel): the f32 results equal the dequantised weights."""
    n, k = 51866, 1280
    rng = np.random.default_rng(29 + m)
    qs, sc = synth.q8_weight(rng, n, k)
    ks = np.array([0, 31, 32, 63, 64, 640, 1247, 1279, 5, 97, 300, 511, 512, 700, 1000, 1200])[:m]
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), ks] = 1.0
    c = _pproj(q, x, qs, sc)
    ref = O.dequant_q8_f16(qs, sc)[ks].astype(np.float32)
    assert np.array_equal(c, ref)


def test_pproj_one_hot_is_dequant(q):
    """x = one-hot rows: out[m][n] = fp16_rne(q s) of column k_m, bit-exact."""
    n, k = 96, 128
    rng = np.random.default_rng(17)
    qs, sc = synth.q8_weight(rng, n, k)
    ks = np.array([0, 1, 31, 32, 63, 64, 100, 127])
    x = np.zeros((len(ks), k), np.float32)
    x[np.arange(len(ks)), ks] = 1.0
    c = _pproj(q, x, qs, sc)
    ref = O.dequant_q8_f16(qs, sc)[ks].astype(np.float32)  # [len(ks)][N]
    assert np.array_equal(c, ref)


# ------------------------------------------------------------------ HIP graph replay
def test_graph_replay_decode_sequence(q):
    """A decode-style launch sequence (batched projection, GEMV, GEMM) captured
    into a HIP graph: every replay, with eager work and synchronisations in
    between, must match the eager results exactly (same kernels, same inputs)."""
    say("graph replay")
    rng = np.random.default_rng(31)
    n1, k1 = 3840, 1280
    qs1, sc1 = synth.q8_weight(rng, n1, k1)
    w1 = q.upload_q8(qs1, sc1)
    qs2, sc2 = synth.q8_weight(rng, 1280, 1280)
    w2 = q.upload_q8(qs2, sc2)
    x = dev(rng.standard_normal((8, k1)).astype(np.float32))
    xv = dev(rng.standard_normal(k1).astype(np.float32))
    a = dev_f16(synth.activations(rng, 300, 1280))
    o1 = torch.empty((8, n1), dtype=torch.float32, device="cuda")
    o2 = torch.empty(1280, dtype=torch.float32, device="cuda")
    c = torch.empty((300, 1280), dtype=torch.int16, device="cuda")

    def seq():
        q.pproj(x, w1, o1, 8, n1, k1)
        q.kGemvQ8(o2, xv, w2, 1280, 1280)
        q.kGemmQ8(a, w2, c, 300, 1280, 1280)

    seq()
    q.sync()
    want = (o1.clone(), o2.clone(), c.clone())
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            q.init(side)
            seq()
    q.init()  # back to the current stream for eager calls
    for rep in range(4):
        for t in (o1, o2):
            t.fill_(float("nan"))
        c.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o1, want[0]) and torch.equal(o2, want[1]) and torch.equal(c, want[2]), rep
        seq()  # eager work between replays
        q.sync()


def test_graph_replay_after_workspace_growth(q):
    """Split-K launches captured while the workspace holds its initial 4 MiB
    (a fresh library: madi_cleanup then madi_init), then an eager split GEMM
    that needs 15.7 MB grows it (1000 x 5120 -> 1280: 80 tiles of 64 x 256,
    three K splits): the outgrown buffer stays allocated, so the graph's
    kernels, which still name it, replay to the eager results."""
    say("graph replay after workspace growth")
    from madi_amd import _lib
    _lib.lib().madi_cleanup()
    q.init()
    rng = np.random.default_rng(37)
    qs1, sc1 = synth.q8_weight(rng, 1280, 5120)     # FFN down: four K splits
    w1 = q.upload_q8(qs1, sc1)
    x = dev(rng.standard_normal((8, 5120)).astype(np.float32))
    xv = dev(rng.standard_normal(5120).astype(np.float32))
    a = dev_f16(synth.activations(rng, 20, 4096))
    qs2, sc2 = synth.q8_weight(rng, 512, 4096)      # 2 tiles x 4 K splits
    w2 = q.upload_q8(qs2, sc2)
    o1 = torch.empty((8, 1280), dtype=torch.float32, device="cuda")
    o2 = torch.empty(1280, dtype=torch.float32, device="cuda")
    c = torch.empty((20, 512), dtype=torch.int16, device="cuda")

    def seq():
        q.pproj(x, w1, o1, 8, 1280, 5120)
        q.kGemvQ8(o2, xv, w1, 1280, 5120)
        q.kGemmQ8(a, w2, c, 20, 512, 4096)

    seq()
    q.sync()
    want = (o1.clone(), o2.clone(), c.clone())
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            q.init(side)
            seq()
    q.init()
    # 1000 x 5120 -> 1280 (three splits of 80 tiles) grows the workspace past 4 MiB
    a3, qs3, sc3 = synth.gemm_case(38, 1000, 1280, 5120)
    w3 = q.upload_q8(qs3, sc3)
    c3 = torch.empty((1000, 1280), dtype=torch.int16, device="cuda")
    q.kGemmQ8(dev_f16(a3), w3, c3, 1000, 1280, 5120)
    q.sync()
    rows = tile_rows(1000)
    assert normwise(host_f16(c3)[rows], O.q8_gemm_rows(a3, qs3, sc3, rows=rows, threads=8)) <= TOL
    for rep in range(3):
        for t in (o1, o2):
            t.fill_(float("nan"))
        c.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o1, want[0]) and torch.equal(o2, want[1]) and torch.equal(c, want[2]), rep
        seq()
        q.sync()


# ------------------------------------------------------------------ load path: quantise, Q8 files
def _knife_edge_weights(rng, n, k):
    """Random f16 rows plus planted blocks: all zero (scale 1.0), exact half
    steps (w / scale = q + 0.5 exactly: round half away from zero), a block
    whose max maps to 127, and subnormal-range values (f16 subnormal scales)."""
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    w[0, 0:32] = 0
    half = np.array([127, 0.5, 1.5, -2.5, 3.5, -126.5, 64.5, -0.5] * 4, np.float32) * 2.0**-7
    w[1, 32:64] = half.astype(np.float16)
    w[2, 0:32] = np.linspace(-1, 1, 32).astype(np.float16)
    w[3, 64:96] = (rng.standard_normal(32) * 1e-6).astype(np.float16)
    return w


@pytest.mark.parametrize("n,k", [(100, 256), (96, 320), (33, 192), (51866, 1280)])
def test_quantize_bit_exact(q, n, k):
    say(f"quantize n={n} k={k}")
    rng = np.random.default_rng(n)
    w = _knife_edge_weights(rng, n, k)
    got = q.quantize(dev_f16(w), n, k)
    q.sync()
    tq = got._keep[0].cpu().numpy()
    ts = got._keep[1].cpu().numpy().view(np.float16)
    uq, us = q.unpack_host(tq, ts, n, k)
    rq, rs = O.quantize_q8(w)
    assert np.array_equal(uq, rq)
    assert np.array_equal(us.view(np.uint16), rs.view(np.uint16))


def test_q8_file_load_equals_f16_quantize(q, tmp_path):
    """The WHASH identity on the device: a weight loaded from a Q8 file (the
    oracle's quantisation written as K.qs / K.scales) and the same weight
    quantised from an F16 file on the GPU are the same panel bytes, and a GEMV
    through it matches the oracle."""
    st = pytest.importorskip("safetensors.numpy")
    from madi_amd import loader
    n, k = 3840, 1280
    rng = np.random.default_rng(41)
    w = _knife_edge_weights(rng, n, k)
    rq, rs = O.quantize_q8(w)
    f16_path, q8_path = tmp_path / "f16.safetensors", tmp_path / "q8.safetensors"
    st.save_file({"dec.qkv": w}, str(f16_path))
    st.save_file({"dec.qkv.qs": rq, "dec.qkv.scales": rs}, str(q8_path))
    a = loader.load(f16_path, "dec.qkv")
    b = loader.load(q8_path, "dec.qkv")
    q.sync()
    assert torch.equal(a._keep[0], b._keep[0].view(torch.uint8).reshape(-1))
    assert torch.equal(a._keep[1], b._keep[1].reshape(-1))
    x = rng.standard_normal(k).astype(np.float32)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    q.kGemvQ8(out, dev(x), a, n, k)
    q.sync()
    assert normwise(out.cpu().numpy(), O.q8_gemv(x, rq, rs, threads=8)) <= 1e-5


# ------------------------------------------------------------------ plain fp16 GEMMs (F16 weights)
@pytest.mark.parametrize("m,n,k", [(50, 64, 96), (8, 3840, 1280), (300, 1280, 1280)])
def test_matmul_f16_alpha_beta(q, m, n, k):
    """mtl_matmul_f16_enc semantics, C = alpha A.B + beta C, against the
    oracle's restatement; MPS's accumulation order is undocumented, so the bar
    is the fp32-accumulation + f16-rounding bound, not bits."""
    say(f"matmul_f16 m={m} n={n} k={k}")
    rng = np.random.default_rng(m + n)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
    c0 = rng.standard_normal((m, n)).astype(np.float16)
    for alpha, beta in ((1.0, 0.0), (0.5, 2.0)):
        dc = dev_f16(c0)
        q.matmulF16Batched(dev_f16(a), dev_f16(b), dc, m, n, k, alpha, beta)
        q.sync()
        got = host_f16(dc).astype(np.float64)
        ref = O.gemm_f16(a, b, c=c0, alpha=alpha, beta=beta, threads=8).astype(np.float64)
        assert normwise(got, ref) <= TOL
        exact = alpha * (a.astype(np.float64) @ b.astype(np.float64)) + beta * c0.astype(np.float64)
        bound = 2.0**-11 * np.abs(exact) + (k + 2) * 2.0**-24 * (
            abs(alpha) * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
            + abs(beta) * np.abs(c0.astype(np.float64))) + 2.0**-24
        assert np.all(np.abs(got - exact) <= bound * 1.001)


@pytest.mark.parametrize("epi", [O.EPI_NONE, O.EPI_BIAS, O.EPI_BIAS_GELU])
def test_f16_gemm_kM4_epilogues(q, epi):
    """kM4 / kM4Bias on an F16 weight produced by kDeq from a Q8 weight: the
    product is rounded to f16 before the bias (m4_gemm.metal:79-85), which
    composes the oracle's f16 GEMM, f32->f16 rounding and GELU."""
    m, n, k = 96, 512, 1280
    a, qs, sc = synth.gemm_case(77, m, n, k)
    w16 = O.dequant_q8_f16(qs, sc)  # [K][N]
    bias = np.random.default_rng(78).standard_normal(n).astype(np.float32)
    dc = torch.empty((m, n), dtype=torch.int16, device="cuda")
    if epi == O.EPI_NONE:
        q.kM4("m4_gemm_nn", dev_f16(a), dev_f16(w16), dc, m, n, k)
    else:
        q.kM4Bias("m4_gemm_bias_gelu" if epi == O.EPI_BIAS_GELU else "m4_gemm_bias",
                  dev_f16(a), dev_f16(w16), dc, dev(bias), m, n, k)
    q.sync()
    got = host_f16(dc).astype(np.float64)
    c16 = O.gemm_f16(a, w16, threads=8)
    if epi == O.EPI_NONE:
        ref = c16.astype(np.float64)
    else:
        v = c16.astype(np.float32) + bias[None, :]
        if epi == O.EPI_BIAS_GELU:
            v = np.vectorize(O.gelu_erf, otypes=[np.float32])(v)
        ref = O.f32_to_f16(v).astype(np.float64)
    assert normwise(got, ref) <= TOL


# kM4 / kM4Bias on true F16 weights (the encoder's F16 cache) through the
# hand-written NN GEMM: each tile shape (128 x 256 from 160 tiles, else
# 128 x 128, else 64 x 128), ragged row counts, K loops shorter than the LDS
# ring (1 and 3 chunks) and fc2's 80 chunks, the encoder's M = 1500 shapes
NN_CASES = [
    (1500, 5120, 1280, O.EPI_BIAS_GELU),  # fc1: 128 x 256 tiles
    (1000, 5120, 1280, O.EPI_NONE),       # 128 x 256, last tile 104 rows
    (1500, 5120, 64, O.EPI_BIAS),         # 128 x 256, one chunk
    (1500, 2560, 1280, O.EPI_NONE),       # cross K|V: 128 x 128 tiles
    (1500, 1280, 1280, O.EPI_BIAS),       # q, k, v, out: 64 x 128 tiles
    (1500, 1280, 5120, O.EPI_NONE),       # fc2: 64 x 128, 80 chunks
    (65, 384, 192, O.EPI_BIAS_GELU),      # three chunks, 65 rows
    (1, 128, 64, O.EPI_BIAS),             # one row, one chunk
    (24000, 5120, 1280, O.EPI_NONE),      # 16 windows: 3760 tiles, 15 rounds
]


@pytest.mark.parametrize("m,n,k,epi", NN_CASES)
def test_f16_nn_gemm(q, m, n, k, epi):
    """The F16-weight GEMM with the reference's epilogue order (the product
    rounded to f16, then + bias, GELU, rounded again; m4_gemm.metal:79-85,
    108-114) against the oracle's f16 GEMM on rows over every 32- and 64-row
    boundary: element-wise within fp32 accumulation + one f16 rounding of the
    exact product (no epilogue), normwise within the path's tolerance of the
    composed oracle (with one)."""
    say(f"f16 NN GEMM m={m} n={n} k={k} epi={epi}")
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
    bias = rng.standard_normal(n).astype(np.float32)
    dc = torch.full((m, n), -1, dtype=torch.int16, device="cuda")
    if epi == O.EPI_NONE:
        q.kM4("m4_gemm_nn", dev_f16(a), dev_f16(b), dc, m, n, k)
    else:
        q.kM4Bias("m4_gemm_bias_gelu" if epi == O.EPI_BIAS_GELU else "m4_gemm_bias",
                  dev_f16(a), dev_f16(b), dc, dev(bias), m, n, k)
    q.sync()
    rows = np.unique(np.r_[0, 1, 31, 32, 63, 64, 127, 128, 255, 256, m // 2, m - 2, m - 1,
                           np.arange(0, m, 1537)])
    rows = rows[(rows >= 0) & (rows < m)]
    got = host_f16(dc)[rows].astype(np.float64)
    c16 = O.gemm_f16(a[rows], b, threads=8)
    if epi == O.EPI_NONE:
        exact = a[rows].astype(np.float64) @ b.astype(np.float64)
        bound = 2.0**-11 * np.abs(exact) + (k + 2) * 2.0**-24 * (
            np.abs(a[rows].astype(np.float64)) @ np.abs(b.astype(np.float64))) + 2.0**-24
        assert np.all(np.abs(got - exact) <= bound * 1.001)
        ref = c16.astype(np.float64)
    else:
        v = c16.astype(np.float32) + bias[None, :]
        if epi == O.EPI_BIAS_GELU:
            v = np.vectorize(O.gelu_erf, otypes=[np.float32])(v)
        ref = O.f32_to_f16(v).astype(np.float64)
    assert normwise(got, ref) <= TOL


def test_f16_nn_gemm_random_shapes(q):
    """Seeded random shapes the NN kernel takes (M any, N a multiple of 128,
    K of 64), each epilogue in turn, element-wise against the oracle on every
    row (fp32 accumulation + f16 rounding bound for the plain product,
    normwise for the epilogues)."""
    rng = np.random.default_rng(2024)
    for t in range(8):
        m = int(rng.integers(1, 400))
        n = 128 * int(rng.integers(1, 17))
        k = 64 * int(rng.integers(1, 25))
        epi = (O.EPI_NONE, O.EPI_BIAS, O.EPI_BIAS_GELU)[t % 3]
        say(f"f16 NN GEMM random m={m} n={n} k={k} epi={epi}")
        a = rng.standard_normal((m, k)).astype(np.float16)
        b = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
        bias = rng.standard_normal(n).astype(np.float32)
        dc = torch.full((m, n), -1, dtype=torch.int16, device="cuda")
        if epi == O.EPI_NONE:
            q.kM4("m4_gemm_nn", dev_f16(a), dev_f16(b), dc, m, n, k)
        else:
            q.kM4Bias("m4_gemm_bias_gelu" if epi == O.EPI_BIAS_GELU else "m4_gemm_bias",
                      dev_f16(a), dev_f16(b), dc, dev(bias), m, n, k)
        q.sync()
        got = host_f16(dc).astype(np.float64)
        c16 = O.gemm_f16(a, b, threads=8)
        if epi == O.EPI_NONE:
            exact = a.astype(np.float64) @ b.astype(np.float64)
            bound = 2.0**-11 * np.abs(exact) + (k + 2) * 2.0**-24 * (
                np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))) + 2.0**-24
            assert np.all(np.abs(got - exact) <= bound * 1.001), (m, n, k)
            ref = c16.astype(np.float64)
        else:
            v = c16.astype(np.float32) + bias[None, :]
            if epi == O.EPI_BIAS_GELU:
                v = np.vectorize(O.gelu_erf, otypes=[np.float32])(v)
            ref = O.f32_to_f16(v).astype(np.float64)
        assert normwise(got, ref) <= TOL, (m, n, k, epi)


@pytest.mark.parametrize("m,n,k,shift", [(8, 5120, 1280, 0), (300, 1280, 1280, 0),
                                         (1500, 5120, 1280, 0), (40, 1280, 1280, 1)])
def test_proj_true_f16_weight(q, m, n, k, shift):
    """proj (decoder.zig:337-341) on a true F16 weight: the activations
    staged to f16 in the caller's in16 buffer, then the NN GEMM with an f32
    result (an output 4 bytes off 16-byte alignment takes rocBLAS instead),
    element-wise within fp32 accumulation of the exact f16 products."""
    say(f"proj on a true F16 weight m={m} n={n} k={k} shift={shift}")
    rng = np.random.default_rng(m + n + shift)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w16 = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
    in16 = torch.empty(m * k, dtype=torch.int16, device="cuda")
    buf = torch.full((m * n + 4,), float("nan"), dtype=torch.float32, device="cuda")
    out = buf[shift:shift + m * n]
    q.proj(in16, dev(x), dev_f16(w16), out, m, n, k)
    q.sync()
    got = out.cpu().numpy().reshape(m, n).astype(np.float64)
    a = x.astype(np.float16).astype(np.float64)
    exact = a @ w16.astype(np.float64)
    bound = (k + 2) * 2.0**-24 * (np.abs(a) @ np.abs(w16.astype(np.float64))) + 2.0**-30
    assert np.all(np.abs(got - exact) <= bound)
    assert np.array_equal(host_f16(in16).reshape(m, k), x.astype(np.float16))


def test_f16_nn_gemm_leaves_other_rows(q):
    """Rows past M are never written (the last tile's clamped rows are read,
    not stored): the output sits inside a taller sentinel buffer."""
    m, n, k = 70, 256, 128
    rng = np.random.default_rng(90)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((k, n)) * 0.05).astype(np.float16)
    big = torch.full((m + 64, n), 0x7E00, dtype=torch.int16, device="cuda")
    q.kM4("m4_gemm_nn", dev_f16(a), dev_f16(b), big, m, n, k)
    q.sync()
    out = big.cpu().numpy()
    assert np.all(out[m:] == 0x7E00)
    assert normwise(out[:m].view(np.float16).astype(np.float64),
                    O.gemm_f16(a, b, threads=8).astype(np.float64)) <= TOL


def test_stream_switch_orders_split_k(q):
    """madi_set_stream makes the new stream wait for the work already issued
    on the old one.  Split-K launches (the FFN-down GEMV 5120 -> 1280, four K
    splits, and the GEMM 1000 x 5120 -> 1280, three K splits through the
    workspace) go to two streams in turn while the first is still busy with
    twenty such GEMMs.  They share the workspace's partials and arrival
    counters one after the other, so every output equals its single-stream
    result bit for bit, round after round (counters left off zero would show
    in the later rounds)."""
    say("stream switch: split-K launches on two streams")
    rng = np.random.default_rng(41)
    qs1, sc1 = synth.q8_weight(rng, 1280, 5120)
    w1 = q.upload_q8(qs1, sc1)
    xs = [dev(rng.standard_normal(5120).astype(np.float32)) for _ in range(4)]
    a = dev_f16(synth.activations(rng, 1000, 5120))
    c = torch.empty((1000, 1280), dtype=torch.int16, device="cuda")
    outs = [torch.empty(1280, dtype=torch.float32, device="cuda") for _ in range(4)]
    q.init()
    for x, o in zip(xs, outs):
        q.kGemvQ8(o, x, w1, 1280, 5120)
    q.kGemmQ8(a, w1, c, 1000, 1280, 5120)
    q.sync()
    want, want_c = [o.clone() for o in outs], c.clone()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        c.fill_(0)
        torch.cuda.synchronize()
        q.init(s1)
        for _ in range(20):
            q.kGemmQ8(a, w1, c, 1000, 1280, 5120)
        q.kGemvQ8(outs[0], xs[0], w1, 1280, 5120)
        q.kGemvQ8(outs[1], xs[1], w1, 1280, 5120)
        q.init(s2)
        q.kGemvQ8(outs[2], xs[2], w1, 1280, 5120)
        q.kGemmQ8(a, w1, c, 1000, 1280, 5120)
        q.init(s1)
        q.kGemvQ8(outs[3], xs[3], w1, 1280, 5120)
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), (rep, i)
        assert torch.equal(c, want_c), rep
    q.init()
