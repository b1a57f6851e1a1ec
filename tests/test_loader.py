"""Q8 weight loading without a GPU: the safetensors reader against files
written here in the reference's Q8 format (K.qs int8 [out][in], K.scales f16
[out][in/32], other tensors copied; engine/metal/bench/quantize_q8.py:42-57),
and the WHASH weight identity against the oracle's FNV-1a restatement."""
import numpy as np
import pytest

import oracle as O
from madi_amd import loader, synth
import madi_amd.q8 as q8

safetensors_numpy = pytest.importorskip("safetensors.numpy")


def _write(path, tensors):
    safetensors_numpy.save_file(tensors, str(path), metadata={"format": "sovereign-q8"})


def test_reads_q8_pairs_and_lists_keys(tmp_path):
    rng = np.random.default_rng(3)
    qa, sa = synth.q8_weight(rng, 96, 128)
    qb, sb = synth.q8_weight(rng, 40, 64)
    f16 = rng.standard_normal((8, 64)).astype(np.float16)
    path = tmp_path / "m.safetensors"
    _write(path, {"enc.fc1.qs": qa, "enc.fc1.scales": sa, "dec.qkv.qs": qb, "dec.qkv.scales": sb,
                  "ln.weight": f16})
    assert loader.q8_keys(path) == ["dec.qkv", "enc.fc1"]
    q, s = loader.read_q8(path, "enc.fc1")
    assert np.array_equal(q, qa) and np.array_equal(s.view(np.uint16), sa.view(np.uint16))
    # the rows a loader reads repack to the documented panel layout and back
    tq, ts = q8.repack_host(q, s)
    uq, us = q8.unpack_host(tq, ts, 96, 128)
    assert np.array_equal(uq, qa) and np.array_equal(us.view(np.uint16), sa.view(np.uint16))


def test_rejects_malformed_q8_tensors(tmp_path):
    rng = np.random.default_rng(4)
    qa, sa = synth.q8_weight(rng, 32, 64)
    path = tmp_path / "bad.safetensors"
    _write(path, {"w.qs": qa, "w.scales": sa[:, :1].copy(), "v.qs": qa.astype(np.int16),
                  "v.scales": sa})
    with pytest.raises(ValueError):
        loader.read_q8(path, "w")
    with pytest.raises(ValueError):
        loader.read_q8(path, "v")


def test_whash_matches_oracle_fnv():
    """madi_q8_fnv (the product's WHASH) against the oracle's FNV-1a, which is
    pinned by the published FNV-1a 64 test vectors; chained over two weights as
    transcribe.zig:1224-1230 chains its five."""
    rng = np.random.default_rng(5)
    w1 = synth.q8_weight(rng, 64, 128)
    w2 = synth.q8_weight(rng, 32, 64)
    x = O.fnv_q8(*w1, seed=O.FNV_SEED)
    x = O.fnv_q8(*w2, seed=x)
    assert loader.whash([w1, w2]) == x
    assert q8.fnv(q8.FNV_SEED, *w1) == O.fnv_q8(*w1)
    # one flipped quant changes the identity
    q_bad = w1[0].copy()
    q_bad[3, 7] ^= 1
    assert loader.whash([(q_bad, w1[1]), w2]) != x
