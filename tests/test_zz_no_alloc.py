"""The allocation-free GEMM entry point (madi_q8_gemm_noalloc) against
madi_q8_gemm through the C ABI: the same kernels, so the results must agree
bit for bit, on two calls in a row (the second smaller, so it runs on what
the first left in the fixed scratch array), and under HIP graph capture,
where the workspace-backed entry point could not grow its buffer."""
import ctypes
import sys

import numpy as np
import pytest

import oracle as O
from madi_amd import _lib, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


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


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16).view(np.int16)).cuda()


def run(q, name, a_d, w, bias_d, m, n, k, epi):
    c = torch.full((m, n), -1, dtype=torch.int16, device="cuda")
    _lib.call(name, a_d.data_ptr(), w.qs, w.scales, c.data_ptr(),
              None if bias_d is None else bias_d.data_ptr(), m, n, k, epi)
    q.sync()
    return c.cpu().numpy()


# (m, n, k, epilogue): 1000 x 5120 -> 1280 + bias (80 tiles of 64 x 256,
# three K splits: 15.7 MB of partials), then smaller split shapes (four
# splits over 25 and 2 tiles), then a shape that does not split at all, and
# fc2 + bias at M = 1500, whose K split stays inside the workgroup (no scratch)
CASES = [(1000, 1280, 5120, _lib.EPI_BIAS), (257, 1280, 5120, _lib.EPI_NONE),
         (20, 512, 4096, _lib.EPI_BIAS_GELU), (96, 512, 1280, _lib.EPI_BIAS_GELU),
         (1500, 1280, 5120, _lib.EPI_BIAS)]


def test_noalloc_matches_gemm_two_calls(q):
    rng = np.random.default_rng(7)
    for i, (m, n, k, epi) in enumerate(CASES):
        say(f"noalloc call {i}: m={m} n={n} k={k} epi={epi}")
        a, qs, sc = synth.gemm_case(100 + i, m, n, k)
        bias = rng.standard_normal(n).astype(np.float32)
        w = q.upload_q8(qs, sc)
        a_d = dev_f16(a)
        b_d = torch.from_numpy(bias).cuda() if epi != _lib.EPI_NONE else None
        got = run(q, "madi_q8_gemm_noalloc", a_d, w, b_d, m, n, k, epi)
        want = run(q, "madi_q8_gemm", a_d, w, b_d, m, n, k, epi)
        assert np.array_equal(got, want), (m, n, k, epi)
        rows = np.unique(np.r_[0, 31, 32, 63, 64, m // 2, m - 1])
        rows = rows[rows < m]
        ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=bias if epi else None,
                             epilogue=epi, threads=8)
        c = got.view(np.float16)[rows].astype(np.float64)
        err = np.max(np.abs(c - ref)) / np.max(np.abs(ref))
        assert err <= 1e-3, err


def test_noalloc_rejects_bad_arguments(q):
    L = _lib.lib()
    rc = L.madi_q8_gemm_noalloc(0x100000, 0x100000, 0x100000, 0x100000, None, 16, 100, 1280, 0)
    assert rc == -5  # n % 32
    rc = L.madi_q8_gemm_noalloc(None, 0x100000, 0x100000, 0x100000, None, 16, 256, 1280, 0)
    assert rc == -6


def test_noalloc_under_graph_capture(q):
    """A fresh library (its growable workspace back at the 4 MiB of madi_init)
    captures 1000 x 5120 -> 1280 + bias: 80 tiles of 64 x 256 with K split
    three ways across workgroups, whose 15.7 MB of fp32 partial tiles and
    arrival counters live in the library's fixed scratch array.  Inside the
    capture, madi_q8_gemm on the same shape is refused (its workspace would
    have to grow, which capture forbids; nothing is launched), so the capture
    needs the allocation-free route.  Every replay, with eager split-K calls
    on the same scratch between them, equals the eager result."""
    m, n, k = 1000, 1280, 5120
    say(f"noalloc graph capture m={m} n={n} k={k}")
    _lib.lib().madi_cleanup()
    q.init()
    a, qs, sc = synth.gemm_case(55, m, n, k)
    bias = np.random.default_rng(56).standard_normal(n).astype(np.float32)
    w = q.upload_q8(qs, sc)
    a_d, b_d = dev_f16(a), torch.from_numpy(bias).cuda()
    c = torch.empty((m, n), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    refused = None
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            q.init(side)
            refused = _lib.lib().madi_q8_gemm(a_d.data_ptr(), w.qs, w.scales, c.data_ptr(),
                                              b_d.data_ptr(), m, n, k, _lib.EPI_BIAS)
            _lib.call("madi_q8_gemm_noalloc", a_d.data_ptr(), w.qs, w.scales, c.data_ptr(),
                      b_d.data_ptr(), m, n, k, _lib.EPI_BIAS)
    q.init()
    assert refused == -9, refused  # MADI_ERR_ARG: the workspace cannot grow under capture
    want = run(q, "madi_q8_gemm", a_d, w, b_d, m, n, k, _lib.EPI_BIAS)
    for rep in range(3):
        c.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy(), want), rep
        # eager work between replays: smaller split shapes through the same
        # scratch (257 rows: four splits over 25 tiles) and the workspace
        a2, qs2, sc2 = synth.gemm_case(57 + rep, 257, 1280, 5120)
        w2 = q.upload_q8(qs2, sc2)
        a2_d = dev_f16(a2)
        assert np.array_equal(run(q, "madi_q8_gemm_noalloc", a2_d, w2, None, 257, 1280, 5120, 0),
                              run(q, "madi_q8_gemm", a2_d, w2, None, 257, 1280, 5120, 0))
    rows = np.unique(np.r_[0, 63, 64, 500, m - 1])
    ref = O.q8_gemm_rows(a, qs, sc, rows=rows, bias=bias, epilogue=_lib.EPI_BIAS, threads=8)
    got = want.view(np.float16)[rows].astype(np.float64)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-3
