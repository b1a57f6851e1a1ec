"""Exact (float64) encoder self-attention and the error bound that the f16
arithmetic of m4_flash_enc (engine/metal/kernels/m4_gemm.metal:268-407) allows
around it.  Shared by the oracle's pin tests (CPU) and the GPU parity tests.

The reference's result is out = f16(sum_j P_j V_j / (sum_j e_j + 1e-6)) with
e_j = exp(s_j - m) for a running reference max m, P_j = f16(e_j), and every
sum in f32; the GPU kernel sums the rounded P_j instead of the e_j.  Against
the exact softmax(Q K^T / 8) V either differs by
  - the f16 rounding of each P_j (relative 2^-11 while e_j is a normal f16,
    absolute 2^-25 below that): at most 2^-11 max|V| with the reference's
    sum, 2^-11 max|V_j - out| <= 2^-11 (max|V| + |out|) with the rounded
    sum, plus n 2^-25 max|V|;
  - the f32 sums over n keys: at most n 2^-24 max|V|;
  - the final f16 rounding: 2^-11 |out|.
"""
import numpy as np

U16 = 2.0 ** -11


def exact_attention(q, k, v, nh):
    """softmax(Q K^T / 8) V per head in float64; q, k, v: [seq][nh*64]."""
    seq = q.shape[0]
    qf, kf, vf = (np.asarray(x, dtype=np.float64).reshape(seq, nh, 64) for x in (q, k, v))
    out = np.empty((seq, nh, 64))
    for hd in range(nh):
        s = qf[:, hd] @ kf[:, hd].T / 8.0
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, hd] = (p @ vf[:, hd]) / p.sum(axis=1, keepdims=True)
    return out.reshape(seq, nh * 64)


def bound(v, exact, nh):
    """Per-element bound on |f16 kernel result - exact| (see module docstring)."""
    seq = v.shape[0]
    vmax = np.abs(np.asarray(v, dtype=np.float64).reshape(seq, nh, 64)).max(axis=(0, 2))
    per_head = vmax * (U16 * 1.01 + seq * 2.0 ** -25 + seq * 2.0 ** -24)
    return np.repeat(per_head, 64)[None, :] + 2.0 * U16 * np.abs(exact) + 1e-7


def within(out, exact, v, nh, factor=1.0):
    """(all elements inside factor x bound, worst ratio |err| / bound)."""
    err = np.abs(np.asarray(out, dtype=np.float64) - exact)
    b = factor * bound(v, exact, nh)
    return bool(np.all(err <= b)), float((err / b).max())


def normwise(out, ref):
    """||out - ref|| / ||ref|| over the whole result."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(out - ref) / np.linalg.norm(ref))
