"""Encoder self-attention (madi_flash_enc_f16, the replacement of m4_flash_enc,
engine/metal/kernels/m4_gemm.metal:268-407) against the oracle and against
float64 softmax attention, through the C ABI.

Bars: every element within the bound the f16 rounding of P allows around the
exact attention (tests/attn_check.py; the kernel's error has the same sources
as the oracle's), within twice that bound of the oracle, and a normwise
relative difference from the oracle under 1e-3.  Every kernel variant (one
to four key groups per workgroup splitting the key range; one and two with the
pipelined schedule, three and four with the plain one) runs every case.
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
from attn_check import exact_attention, normwise, within
from madi_amd import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def q8():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import madi_amd.q8 as q8
    q8.init()
    return q8


@pytest.fixture(params=[1, 2, 3, 4], ids=["one_group", "two_groups", "three_groups", "four_groups"])
def ksplit(request):
    old = os.environ.get("MADI_FLASH_KSPLIT")
    os.environ["MADI_FLASH_KSPLIT"] = str(request.param)
    yield request.param
    if old is None:
        os.environ.pop("MADI_FLASH_KSPLIT", None)
    else:
        os.environ["MADI_FLASH_KSPLIT"] = old


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16).view(np.int16)).cuda()


def host_f16(t):
    return t.cpu().numpy().view(np.float16)


def qkv(rng, seq, nh, scale=1.0, dist="normal"):
    shape = (seq, nh * 64)
    if dist == "uniform":  # engine/metal/test_m4.zig:87-89
        return [((rng.random(shape) - 0.5) * 2.0).astype(np.float16) for _ in range(3)]
    return [(rng.standard_normal(shape) * scale).astype(np.float16) for _ in range(3)]


def run(q8, q, k, v, nh, out=None):
    seq = q.shape[0]
    tq, tk, tv = dev_f16(q), dev_f16(k), dev_f16(v)
    to = torch.empty_like(tq) if out is None else out
    _lib.call("madi_flash_enc_f16", to.data_ptr(), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
              seq, nh)
    torch.cuda.synchronize()
    return host_f16(to)


def check(got, q, k, v, nh):
    assert np.all(np.isfinite(got.astype(np.float32)))
    exact = exact_attention(q, k, v, nh)
    ok, worst = within(got, exact, v, nh)
    assert ok, f"vs fp64: worst |err|/bound {worst:.3f}"
    ref = O.flash_enc_f16(q, k, v, nh, threads=16)
    ok, worst = within(got, ref.astype(np.float64), v, nh, factor=2.0)
    assert ok, f"vs oracle: worst |err|/(2 bound) {worst:.3f}"
    err = normwise(got, ref)
    assert err <= 1e-3, err
    return err


CASES = [
    (1, 1, 1.0, "normal"), (5, 2, 1.0, "normal"), (63, 1, 1.0, "normal"),
    (64, 2, 1.0, "normal"), (65, 1, 1.0, "normal"), (127, 2, 2.0, "normal"),
    (128, 1, 1.0, "normal"), (129, 3, 1.0, "normal"), (200, 2, 3.0, "normal"),
    (257, 2, 1.0, "uniform"), (700, 4, 2.0, "normal"),
]


@pytest.mark.parametrize("seq,nh,scale,dist", CASES)
def test_flash_vs_oracle(q8, ksplit, seq, nh, scale, dist):
    """Single and multi-block key ranges, ragged query and key tails (1 row,
    63/64/65, 127/128/129), flat and sharp softmax (scale 2-3: the reference
    max moves between blocks)."""
    say(f"flash seq={seq} nh={nh} scale={scale} {dist} groups={ksplit}")
    rng = np.random.default_rng(seq * 31 + nh)
    q, k, v = qkv(rng, seq, nh, scale, dist)
    check(run(q8, q, k, v, nh), q, k, v, nh)


def test_flash_encoder_window(q8, ksplit):
    """The encoder's shape, 1500 frames x 20 heads, on the reference test's
    uniform(-1, 1) inputs (engine/metal/test_m4.zig:78-134, whose own bar is
    |diff| <= 0.01 between its two kernels)."""
    say(f"flash 1500x20 uniform groups={ksplit}")
    rng = np.random.default_rng(23)
    q, k, v = qkv(rng, 1500, 20, dist="uniform")
    got = run(q8, q, k, v, 20)
    check(got, q, k, v, 20)
    ref = O.flash_enc_f16(q, k, v, 20, threads=16)
    assert np.abs(got.astype(np.float32) - ref.astype(np.float32)).max() <= 0.01


def test_flash_reruns_bit_identical_and_in_place(q8):
    """Deterministic: two runs agree bit for bit; out == q (each query row is
    read before its output is written) gives the same result."""
    say("flash reruns / in place")
    rng = np.random.default_rng(7)
    seq, nh = 1500, 20
    q, k, v = qkv(rng, seq, nh)
    a = run(q8, q, k, v, nh)
    b = run(q8, q, k, v, nh)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    tq, tk, tv = dev_f16(q), dev_f16(k), dev_f16(v)
    _lib.call("madi_flash_enc_f16", tq.data_ptr(), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(),
              seq, nh)
    torch.cuda.synchronize()
    assert np.array_equal(host_f16(tq).view(np.uint16), a.view(np.uint16))


def test_flash_closed_forms(q8):
    """q = 0: uniform weights, out = the mean of the value rows; q_i = 16 k_pi(i):
    out_i = V_pi(i) to one f16 ulp."""
    say("flash closed forms")
    rng = np.random.default_rng(9)
    seq, nh = 700, 2
    _, k, v = qkv(rng, seq, nh)
    got = run(q8, np.zeros_like(k), k, v, nh).astype(np.float64)
    mean = v.astype(np.float64).mean(axis=0)
    ulp = np.spacing(np.abs(mean).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - mean[None, :]) <= ulp[None, :] + seq * 2.0 ** -24 * np.abs(v).max())
    perm = rng.permutation(seq)
    qa = (16.0 * k[perm].astype(np.float32)).astype(np.float16)
    got = run(q8, qa, k, v, nh).astype(np.float64)
    assert np.all(np.abs(got - v[perm].astype(np.float64)) <= np.spacing(np.abs(v[perm])))


def test_flash_seq_zero_and_errors(q8):
    rng = np.random.default_rng(1)
    q, k, v = qkv(rng, 64, 1)
    tq, tk, tv = dev_f16(q), dev_f16(k), dev_f16(v)
    to = dev_f16(np.full_like(q, 7.0))
    L = _lib.lib()
    assert L.madi_flash_enc_f16(to.data_ptr(), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 0, 1) == 0
    torch.cuda.synchronize()
    assert np.all(host_f16(to) == 7.0)
    assert L.madi_flash_enc_f16(tk.data_ptr(), tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 64, 1) == -9
    assert L.madi_flash_enc_f16(to.data_ptr() + 2, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 64, 1) == -7
