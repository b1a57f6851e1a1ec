"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so that a plausible mistake in the restatement (a wrong
scale index, a dropped or extra term, a transposed operand, fused multiply-add
contraction, the wrong rounding mode) fails it.  The oracle is never compared
with a copy of its own formula only: the anchors are independent
implementations (numpy's float16, math.erf, exact fp64/integer arithmetic),
closed forms, published test vectors and brute force on tiny inputs.
"""
import math

import numpy as np
import pytest

import oracle as O


# ---------------------------------------------------------------- fp16 <-> fp32
def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    got = O.f16_to_f32(h)
    ref = h.astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_vs_numpy():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    # knife edges: exact ties at every f16 exponent, subnormal boundaries, overflow
    ties = []
    for e in range(-24, 16):
        base = np.float32(2.0) ** e
        for m in (1, 3, 5, 1023, 1025):
            ties.append(base * (1 + (m + 0.5) / 1024))
    extra = np.array(ties + [65504, 65519.996, 65520, 65536, 2**-24, 2**-25, 1.5 * 2**-25,
                             2**-14, 2**-14 - 2**-25, 0.0, -0.0, np.inf, -np.inf],
                     dtype=np.float32)
    f = np.concatenate([f, extra, -extra])
    got = O.f32_to_f16(f)
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint16), ref[~nan].view(np.uint16))


# ---------------------------------------------------------------- dequant
def _all_f16_in(lo, hi):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = h.astype(np.float32)
    return h[(f >= lo) & (f <= hi)]


def test_dequant_exhaustive_grid():
    """All 255 q values x every fp16 scale in [1e-3, 1e-2], plus subnormal and
    large scales: f16(f32(q) * f32(s)) must equal numpy's fp16 multiply of the
    exact operands (one correctly rounded IEEE product), element for element,
    and land at out[k][n] (the transposed [K][N] layout)."""
    scales = np.concatenate([_all_f16_in(1e-3, 1e-2),
                             np.array([2**-24, 3 * 2**-24, 2**-14, 1e-5, 0.25, 1.0, 7.5, 300.0],
                                      dtype=np.float16)])
    q = np.arange(-127, 128, dtype=np.int8)
    n = scales.size
    k = 256  # 8 blocks; block b of row n uses scale (n + b) mod n_scales
    qs = np.empty((n, k), dtype=np.int8)
    qs[:, :255] = q[None, :]
    qs[:, 255] = 0
    sc = np.empty((n, k // 32), dtype=np.float16)
    for b in range(k // 32):
        sc[:, b] = np.roll(scales, -b)
    out = O.dequant_q8_f16(qs, sc)
    assert out.shape == (k, n)
    s_full = np.repeat(sc, 32, axis=1)  # [n][k]
    ref = (qs.astype(np.float16) * s_full)  # numpy f16 multiply: correctly rounded
    assert np.array_equal(out.T.view(np.uint16), ref.view(np.uint16))
    # the f32 route (the reference's own expression) agrees
    ref32 = (qs.astype(np.float32) * s_full.astype(np.float32)).astype(np.float16)
    assert np.array_equal(out.T.view(np.uint16), ref32.view(np.uint16))


# ---------------------------------------------------------------- GEMM
def _q8(rng, n, k):
    qs = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    sc = rng.uniform(1e-3, 1e-2, size=(n, k // 32)).astype(np.float16)
    return qs, sc


def _w64(qs, sc):
    return qs.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=1)


def _fp64_bound_ok(c, a, qs, sc):
    """|c - exact| <= K * 2^-24 * sum|a||w| + tiny: the recursive-summation error
    bound.  A wrong index or a dropped term violates it by orders of magnitude."""
    a64 = a.astype(np.float64)
    w = _w64(qs, sc)
    exact = a64 @ w.T
    bound = a.shape[1] * 2.0**-24 * (np.abs(a64) @ np.abs(w).T) + 1e-30
    return np.all(np.abs(c.astype(np.float64) - exact) <= bound), exact


def test_gemm_fp64_error_bound():
    rng = np.random.default_rng(7)
    m, n, k = 37, 96, 320
    a = rng.standard_normal((m, k)).astype(np.float16)
    qs, sc = _q8(rng, n, k)
    c = O.q8_gemm_rows(a, qs, sc, threads=4)
    ok, exact = _fp64_bound_ok(c, a, qs, sc)
    assert ok
    # and it is not trivially loose: the error is tiny relative to the values
    assert np.max(np.abs(c - exact)) / np.max(np.abs(exact)) < 1e-5


def test_gemm_bound_rejects_planted_mistakes():
    """Planted mistakes, applied to the oracle's inputs on the CPU: each plausible
    slip (neighbour scale block, transposed block order, a dropped final k, a
    sign flip) must be caught by the fp64 bound used above."""
    rng = np.random.default_rng(8)
    m, n, k = 16, 64, 128
    a = rng.standard_normal((m, k)).astype(np.float16)
    qs, sc = _q8(rng, n, k)
    mutants = {
        "scale_of_next_block": (qs, np.roll(sc, 1, axis=1)),
        "dropped_last_k": (np.concatenate([qs[:, :-1], np.zeros((n, 1), np.int8)], 1), sc),
        "row_swapped": (qs[np.r_[1, 0, 2:n]], sc[np.r_[1, 0, 2:n]]),
        "negated_q": (-qs, sc),
    }
    for name, (mq, ms) in mutants.items():
        c_bad = O.q8_gemm_rows(a, mq, ms)
        ok, _ = _fp64_bound_ok(c_bad, a, qs, sc)
        assert not ok, name


def test_gemm_single_block_closed_form():
    """K = 32: C = s * sum(a*q); sum(a*q) of f16 a and integer q is exact in fp64."""
    rng = np.random.default_rng(9)
    m, n, k = 20, 40, 32
    a = rng.standard_normal((m, k)).astype(np.float16)
    qs, sc = _q8(rng, n, k)
    c = O.q8_gemm_rows(a, qs, sc)
    exact = (a.astype(np.float64) @ qs.astype(np.float64).T) * sc.astype(np.float64).T
    assert np.max(np.abs(c - exact)) <= 32 * 2.0**-24 * np.max(np.abs(exact)) * 4


def test_gemm_one_hot_reproduces_dequant_bits():
    """One-hot A row m selecting k(m): C[m][n] = deq(w[n][k(m)]) exactly, and the
    f16 output equals the dequantised weight's bits."""
    rng = np.random.default_rng(10)
    n, k = 64, 96
    qs, sc = _q8(rng, n, k)
    ks = np.arange(k)
    a = np.zeros((k, k), dtype=np.float16)
    a[ks, ks] = 1.0
    c16 = O.q8_gemm_f16(a, qs, sc)
    deq = O.dequant_q8_f16(qs, sc)  # [K][N]
    assert np.array_equal(c16.view(np.uint16), deq.view(np.uint16))


def test_gemm_all_ones_row_sums():
    rng = np.random.default_rng(11)
    n, k = 32, 128
    qs, sc = _q8(rng, n, k)
    a = np.ones((3, k), dtype=np.float16)
    c = O.q8_gemm_rows(a, qs, sc)
    sums = _w64(qs, sc).sum(axis=1)
    assert np.allclose(c, sums[None, :], rtol=0, atol=k * 2.0**-24 * np.abs(_w64(qs, sc)).sum(1).max())


def test_gemm_bruteforce_reference_case_bit_exact():
    """The reference's correctness shape M=50, N=64, K=96 (test_q8gemm.zig:42),
    restated as a pure-Python loop with numpy float32 scalars: bit-identical
    k-sequential fp32 rounding, no contraction."""
    rng = np.random.default_rng(12)
    m, n, k = 50, 64, 96
    a = rng.uniform(-1, 1, size=(m, k)).astype(np.float16)
    qs, sc = _q8(rng, n, k)
    c = O.q8_gemm_rows(a, qs, sc)
    a32 = a.astype(np.float32)
    w32 = qs.astype(np.float32) * np.repeat(sc.astype(np.float32), 32, axis=1)
    for mm in range(0, m, 7):
        for nn in range(0, n, 5):
            acc = np.float32(0)
            for kk in range(k):
                acc = np.float32(acc + np.float32(a32[mm, kk] * w32[nn, kk]))
            assert c[mm, nn] == acc


def test_gemm_row_subset_and_f16_store():
    rng = np.random.default_rng(13)
    m, n, k = 33, 64, 64
    a = rng.standard_normal((m, k)).astype(np.float16)
    qs, sc = _q8(rng, n, k)
    bias = rng.standard_normal(n).astype(np.float32)
    full = O.q8_gemm_rows(a, qs, sc, bias=bias, epilogue=O.EPI_BIAS_GELU, threads=3)
    rows = np.array([32, 0, 17], dtype=np.uint32)
    sub = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=bias, epilogue=O.EPI_BIAS_GELU)
    assert np.array_equal(sub, full[rows])
    c16 = O.q8_gemm_f16(a, qs, sc, bias=bias, epilogue=O.EPI_BIAS_GELU, threads=2)
    assert np.array_equal(c16.view(np.uint16), full.astype(np.float16).view(np.uint16))
    # bias epilogue adds exactly the f32 bias after accumulation
    plain = O.q8_gemm_rows(a, qs, sc)
    withb = O.q8_gemm_rows(a, qs, sc, bias=bias, epilogue=O.EPI_BIAS)
    assert np.array_equal(withb, (plain + bias[None, :]).astype(np.float32))


# ---------------------------------------------------------------- GELU
def test_gelu_erf_against_math_erf():
    xs = np.concatenate([np.linspace(-10, 10, 4001), [0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0]])
    for x in xs:
        x32 = float(np.float32(x))
        exact = 0.5 * x32 * (1.0 + math.erf(x32 / math.sqrt(2.0)))
        got = O.gelu_erf(x32)
        # A&S 7.1.26: |erf error| <= 1.5e-7; the fp32 steps (1 - poly*ex near 1)
        # add a few ulp(1) = 6e-8 each
        assert abs(got - exact) <= 0.5 * abs(x32) * (1.5e-7 + 3e-7) + 4e-7 * abs(exact) + 1e-37, x


# ---------------------------------------------------------------- GEMV
def test_gemv_bound_and_epilogues():
    rng = np.random.default_rng(14)
    n, k = 96, 512
    x = rng.standard_normal(k).astype(np.float32)
    qs, sc = _q8(rng, n, k)
    bias = rng.standard_normal(n).astype(np.float32)
    y = O.q8_gemv(x, qs, sc, threads=2)
    w = _w64(qs, sc)
    exact = w @ x.astype(np.float64)
    bound = k * 2.0**-24 * (np.abs(w) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - exact) <= bound)
    assert np.array_equal(O.q8_gemv(x, qs, sc, bias, O.EPI_BIAS), (y + bias).astype(np.float32))
    g = O.q8_gemv(x, qs, sc, bias, O.EPI_BIAS_GELU)
    assert np.array_equal(g, np.array([O.gelu_erf(float(v)) for v in (y + bias)], np.float32))
    res0 = rng.standard_normal(n).astype(np.float32)
    r = O.q8_gemv(x, qs, sc, bias, O.EPI_BIAS_RES, out=res0)
    assert np.array_equal(r, ((res0 + y) + bias).astype(np.float32))


def test_gemv_qkv_routing():
    rng = np.random.default_rng(15)
    d = 64
    x = rng.standard_normal(d).astype(np.float32)
    qs, sc = _q8(rng, 3 * d, d)
    qb = rng.standard_normal(d).astype(np.float32)
    vb = rng.standard_normal(d).astype(np.float32)
    kc = np.full((5, d), 7.0, np.float32)
    vc = np.full((5, d), 9.0, np.float32)
    q, kc2, vc2 = O.q8_gemv_qkv(x, qs, sc, qb, vb, kc, vc, pos=3)
    y = O.q8_gemv(x, qs, sc)
    assert np.array_equal(q, y[:d] + qb)
    assert np.array_equal(kc2[3], y[d:2 * d])             # k: no bias
    assert np.array_equal(vc2[3], y[2 * d:] + vb)         # v: + vb
    untouched = np.r_[0:3, 4]
    assert np.all(kc2[untouched] == 7.0) and np.all(vc2[untouched] == 9.0)


def test_proj_matches_gemv_rows():
    rng = np.random.default_rng(16)
    m, n, k = 5, 64, 128
    xr = rng.standard_normal((m, k)).astype(np.float32)
    qs, sc = _q8(rng, n, k)
    p = O.q8_proj(xr, qs, sc, threads=2)
    for i in range(m):
        assert np.array_equal(p[i], O.q8_gemv(xr[i], qs, sc))


# ---------------------------------------------------------------- quantiser
def test_quantize_knife_edges_round_half_away():
    # one block whose max is 127 -> scale exactly 1.0, so q = round_half_away(w)
    w = np.zeros((1, 32), np.float32)
    w[0, 0] = 127.0
    w[0, 1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5]
    qs, sc = O.quantize_q8(w.astype(np.float16))
    assert sc[0, 0] == np.float16(1.0)
    assert list(qs[0, :9]) == [127, 3, -3, 1, -1, 2, -2, 127, -127]


def test_quantize_properties():
    rng = np.random.default_rng(17)
    w = (rng.standard_normal((64, 256)) * rng.uniform(1e-3, 2, size=(64, 1))).astype(np.float16)
    w[3, 32:64] = 0  # an all-zero block -> scale 1.0, q = 0
    qs, sc = O.quantize_q8(w)
    assert sc[3, 1] == np.float16(1.0) and np.all(qs[3, 32:64] == 0)
    assert np.all(np.abs(qs.astype(np.int32)) <= 127)
    blocks = np.abs(qs.astype(np.int32)).reshape(64, 8, 32).max(axis=2)
    nz = np.abs(w.astype(np.float32)).reshape(64, 8, 32).max(axis=2) > 0
    assert np.all(blocks[nz] == 127)
    # reconstruction with the f32 scale is within half a step
    wf = w.astype(np.float32).reshape(64, 8, 32)
    mx = np.abs(wf).max(axis=2, keepdims=True)
    s32 = np.where(mx > 0, mx / np.float32(127), np.float32(1))
    err = np.abs(qs.astype(np.float32).reshape(64, 8, 32) * s32 - wf)
    assert np.all(err <= s32 * 0.5 * (1 + 1e-5))
    # odd symmetry
    qn, scn = O.quantize_q8(-w)
    assert np.array_equal(qn, -qs) and np.array_equal(scn, sc)


# ---------------------------------------------------------------- FNV-1a / rows
def test_fnv1a64_published_vectors():
    assert O.fnv1a64(b"") == 0xCBF29CE484222325
    assert O.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert O.fnv1a64(b"foobar") == 0x85944171F73967E8


def test_fnv_q8_is_bytes_then_scales():
    rng = np.random.default_rng(18)
    qs, sc = _q8(rng, 4, 64)
    h = O.fnv_q8(qs, sc)
    assert h == O.fnv1a64(qs.tobytes() + sc.astype("<f2").tobytes())
    qs2 = qs.copy()
    qs2[2, 5] ^= 1
    assert O.fnv_q8(qs2, sc) != h


def test_emb_row_is_f32_dequant():
    rng = np.random.default_rng(19)
    qs, sc = _q8(rng, 10, 64)
    row = O.emb_row_q8(qs, sc, 7)
    ref = qs[7].astype(np.float32) * np.repeat(sc[7].astype(np.float32), 32)
    assert np.array_equal(row, ref)


def test_emb_pe_rows_is_row_plus_position():
    """emb_pe_rows_q8 = the f32 dequantised row (exact: 8 x 11 significant
    bits) plus the positional row, one f32 rounding; with zero positions it
    is the embedding row itself, with zero quants the positional row."""
    rng = np.random.default_rng(23)
    qs, sc = _q8(rng, 12, 128)
    pe = rng.standard_normal((40, 128)).astype(np.float32)
    toks = np.array([3, 0, 11, 3, 7], np.uint32)
    got = O.emb_pe_rows_q8(qs, sc, toks, pe, 30)
    for m, t in enumerate(toks):
        row = qs[t].astype(np.float64) * np.repeat(sc[t].astype(np.float64), 32)
        assert np.array_equal(got[m], (row + pe[30 + m].astype(np.float64)).astype(np.float32))
    assert np.array_equal(O.emb_pe_rows_q8(qs, sc, toks, np.zeros_like(pe), 30)[2],
                          O.emb_row_q8(qs, sc, 11))
    assert np.array_equal(O.emb_pe_rows_q8(np.zeros_like(qs), sc, toks, pe, 1), pe[1:6])


def test_gemm_f16_alpha_beta():
    rng = np.random.default_rng(20)
    m, n, k = 9, 24, 40
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = rng.standard_normal((k, n)).astype(np.float16)
    c0 = rng.standard_normal((m, n)).astype(np.float16)
    c = O.gemm_f16(a, b)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(c.astype(np.float64) - exact)) <= np.max(np.abs(exact)) * 2**-10
    c2 = O.gemm_f16(a, b, c=c0, alpha=0.5, beta=2.0)
    exact2 = 0.5 * exact + 2.0 * c0.astype(np.float64)
    assert np.max(np.abs(c2.astype(np.float64) - exact2)) <= np.max(np.abs(exact2)) * 2**-10
