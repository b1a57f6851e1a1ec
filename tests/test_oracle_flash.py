"""Pins the oracle's encoder self-attention (oracle_flash_enc_f16, the
restatement of m4_flash_enc, engine/metal/kernels/m4_gemm.metal:268-407)
before the GPU kernel is compared with it.

Anchors: float64 softmax attention within the bound the f16 rounding of P
allows (tests/attn_check.py), closed forms (q = 0 gives the mean of the value
rows; a query aligned with one key returns that key's value row), invariances
(joint permutation of keys and values, heads computed independently), and
planted mistakes that the bound must reject.  The reference's own test of
this kernel (engine/metal/test_m4.zig:76-134) compares two of its GPU kernels
with each other at 1500 rows x 20 heads on uniform(-1, 1) inputs and holds no
vectors; its input distribution is one of the cases below.
"""
import numpy as np
import pytest

import oracle as O
from attn_check import exact_attention, within


def _qkv(rng, seq, nh, scale=1.0, dist="normal"):
    shape = (seq, nh * 64)
    if dist == "uniform":  # test_m4.zig:87-89
        return [((rng.random(shape) - 0.5) * 2.0).astype(np.float16) for _ in range(3)]
    return [(rng.standard_normal(shape) * scale).astype(np.float16) for _ in range(3)]


@pytest.mark.parametrize("seq,nh,scale,dist", [
    (1, 1, 1.0, "normal"), (5, 2, 1.0, "normal"), (64, 1, 1.0, "normal"),
    (65, 2, 1.0, "normal"), (200, 3, 1.0, "normal"), (450, 2, 2.0, "normal"),
    (333, 2, 1.0, "uniform"), (130, 1, 3.0, "normal"),
])
def test_flash_oracle_vs_fp64(seq, nh, scale, dist):
    """Single and multi-block key ranges, ragged tails, sharp (scale 2-3:
    scores of std 4-9, the running max moves between blocks) and flat softmax."""
    rng = np.random.default_rng(seq * 7 + nh)
    q, k, v = _qkv(rng, seq, nh, scale, dist)
    out = O.flash_enc_f16(q, k, v, nh, threads=4)
    ok, worst = within(out, exact_attention(q, k, v, nh), v, nh)
    assert ok, worst


def test_flash_oracle_uniform_weights_give_the_mean():
    """q = 0: every score is 0, every e is exactly 1, P = 1, the sum is the key
    count: out = f16(sum_j V_j / (n + 1e-6)), the f32 column sum of V up to its
    rounding."""
    rng = np.random.default_rng(3)
    seq, nh = 300, 2
    _, k, v = _qkv(rng, seq, nh)
    q = np.zeros_like(k)
    out = O.flash_enc_f16(q, k, v, nh).astype(np.float64)
    mean = v.astype(np.float64).sum(axis=0) / (seq + 1e-6)
    ulp = np.spacing(np.abs(mean).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(out - mean[None, :]) <= ulp[None, :] + seq * 2.0 ** -24 * np.abs(v).max())


def test_flash_oracle_aligned_query_returns_that_value_row():
    """q_i = 16 k_pi(i): the matching score (2 |k|^2, about 128) exceeds every
    other by about 90, the other weights (below e^-80) vanish in f16, so
    out_i = V_pi(i) up to one f16 ulp."""
    rng = np.random.default_rng(4)
    seq, nh = 150, 1
    _, k, v = _qkv(rng, seq, nh)
    perm = rng.permutation(seq)
    q = (16.0 * k[perm].astype(np.float32)).astype(np.float16)
    out = O.flash_enc_f16(q, k, v, nh).astype(np.float64)
    want = v[perm].astype(np.float64)
    ulp = np.spacing(np.abs(v[perm])).astype(np.float64)
    assert np.all(np.abs(out - want) <= ulp)


def test_flash_oracle_key_order_and_head_independence():
    rng = np.random.default_rng(5)
    seq, nh = 257, 2
    q, k, v = _qkv(rng, seq, nh)
    out = O.flash_enc_f16(q, k, v, nh)
    perm = rng.permutation(seq)
    out_p = O.flash_enc_f16(q, k[perm], v[perm], nh)
    ok, worst = within(out_p, out.astype(np.float64), v, nh, factor=2.0)
    assert ok, worst
    # head 1's keys and values do not reach head 0's output, bit for bit
    k2, v2 = k.copy(), v.copy()
    k2[:, 64:] = rng.standard_normal((seq, 64)).astype(np.float16)
    v2[:, 64:] = rng.standard_normal((seq, 64)).astype(np.float16)
    out2 = O.flash_enc_f16(q, k2, v2, nh)
    assert np.array_equal(out2[:, :64].view(np.uint16), out[:, :64].view(np.uint16))
    assert not np.array_equal(out2[:, 64:], out[:, 64:])


def test_flash_bound_rejects_planted_mistakes():
    """Plausible slips, planted in the oracle's inputs on the CPU: the 1/8 score
    scale dropped, Q and K swapped (S^T), a sign flip of the scores, values
    misaligned with their keys by one row, the wrong head's values, and padded
    keys left unmasked (zero rows taking part in the softmax).  The fp64 bound
    must reject every one."""
    rng = np.random.default_rng(6)
    seq, nh = 200, 2
    q, k, v = _qkv(rng, seq, nh)
    exact = exact_attention(q, k, v, nh)
    pad = 256 - seq
    zpad = np.zeros((pad, nh * 64), np.float16)
    mutants = {
        "scale_dropped": lambda: O.flash_enc_f16((q.astype(np.float32) * 8).astype(np.float16), k, v, nh),
        "q_k_swapped": lambda: O.flash_enc_f16(k, q, v, nh),
        "scores_negated": lambda: O.flash_enc_f16(-q, k, v, nh),
        "values_shifted": lambda: O.flash_enc_f16(q, k, np.roll(v, 1, axis=0), nh),
        "wrong_head": lambda: O.flash_enc_f16(q, k, np.roll(v, 64, axis=1), nh),
        "tail_unmasked": lambda: O.flash_enc_f16(np.vstack([q, zpad]), np.vstack([k, zpad]),
                                                 np.vstack([v, zpad]), nh)[:seq],
    }
    for name, run in mutants.items():
        ok, _ = within(run(), exact, v, nh)
        assert not ok, name
