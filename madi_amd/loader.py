"""Q8 weight loading: the on-disk half of the load path.

The reference's Q8 model file (engine/metal/bench/quantize_q8.py:42-57) stores
each quantised weight K as two tensors, K.qs (int8 [out][in]) and K.scales
(f16 [out][in/32]), and copies every other tensor unchanged; the engine reads
them with readQ8 (engine/metal/transcribe.zig:327-341) and otherwise quantises
the F16 tensor K at load (quantInto, :309-326).  Here:

  read_q8(path, key)          the natural Q8 rows of K from a Q8 file
  load(path, key)             K as a panel-layout device weight: read K.qs /
                              K.scales and repack, or, for an F16 file,
                              upload K and quantise it on the GPU
  whash(weights)              the WHASH identity (transcribe.zig:1219-1232)
                              over natural-layout weights

Files are read with safetensors' numpy loader, which parses the header and
copies raw tensor bytes only (nothing in the file is executed).
"""
from __future__ import annotations

import numpy as np

from . import q8 as _q8


def _open(path):
    from safetensors import safe_open
    return safe_open(path, framework="numpy")


def q8_keys(path) -> list[str]:
    """Base names K that have both K.qs and K.scales in the file."""
    with _open(path) as f:
        names = set(f.keys())
    return sorted(n[:-3] for n in names if n.endswith(".qs") and n[:-3] + ".scales" in names)


def read_q8(path, key: str):
    """(qs int8 [out][in], scales f16 [out][in/32]) of weight `key`, natural layout."""
    with _open(path) as f:
        qs = f.get_tensor(key + ".qs")
        sc = f.get_tensor(key + ".scales")
    if qs.dtype != np.int8 or qs.ndim != 2:
        raise ValueError(f"{key}.qs: expected a 2-D int8 tensor, got {qs.dtype} {qs.shape}")
    out_ch, in_ch = qs.shape
    if in_ch % 32 or sc.dtype != np.float16 or sc.shape != (out_ch, in_ch // 32):
        raise ValueError(f"{key}.scales: expected f16 [{out_ch}][{in_ch // 32}], got {sc.dtype} {sc.shape}")
    return qs, sc


def load(path, key: str, device="cuda") -> "_q8.Q8":
    """Weight `key` as a panel-layout Q8 device weight.  A Q8 file's K.qs /
    K.scales are repacked on the host and uploaded (readQ8 + repack); an F16
    file's K is uploaded and quantised on the GPU (quantInto + repack, bit-
    identical to what the Q8 file holds for the same F16 source)."""
    with _open(path) as f:
        names = set(f.keys())
        if key + ".qs" in names:
            f_has_q8 = True
        elif key in names:
            f_has_q8 = False
            w = f.get_tensor(key)
        else:
            raise KeyError(f"{key}: neither {key}.qs nor an F16 tensor in {path}")
    if f_has_q8:
        qs, sc = read_q8(path, key)
        return _q8.upload_q8(qs, sc, device=device)
    if w.dtype != np.float16 or w.ndim != 2 or w.shape[1] % 64:
        raise ValueError(f"{key}: expected a 2-D f16 tensor with in % 64 == 0, got {w.dtype} {w.shape}")
    import torch
    n, k = w.shape
    dw = torch.from_numpy(np.ascontiguousarray(w).view(np.int16)).to(device)
    out = _q8.quantize(dw, n, k, device=device)
    out._keep = out._keep + (dw,)
    return out


def whash(weights) -> int:
    """FNV-1a 64 chain over natural-layout (qs, scales) pairs in order, from
    the seed transcribe.zig:1225 starts at."""
    x = _q8.FNV_SEED
    for qs, sc in weights:
        x = _q8.fnv(x, qs, sc)
    return x


__all__ = ["q8_keys", "read_q8", "load", "whash"]
