"""The engine's call sequences, unchanged, through the C ABI.

The encoder's forward pass (engine/metal/encoder.zig:262-301) dequantises
every Q8 weight into a shared F16 scratch (kDeq -> s.wdq / s.wdq2) and
multiplies by it through handles resolved by name (kM4 / kM4Bias with
m4_gemm_nn, m4_gemm_bias, m4_gemm_bias_gelu).  The batched decoder keeps F16
copies made by deqW16 and projects through them (proj, decoder.zig:337-341).
These tests replay those sequences verbatim through the Python mirror of the
wrappers and check that the fused Q8 kernels ran (the F16 scratch is never
written: it still holds a NaN sentinel) with results matching the oracle, and
that the deferred dequantisation is written out wherever anything could
observe it."""
import ctypes
import sys

import numpy as np
import pytest

import oracle as O
from madi_amd import _lib, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-3
D, MLP, M = 1280, 5120, 1500
NAN16 = np.uint16(0x7E00)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def q():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import madi_amd.q8 as q8
    q8.init()
    q8.set_deferred_dequant(True)
    return q8


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def dev_f16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16).view(np.int16)).cuda()


def host_f16(t):
    return t.cpu().numpy().view(np.float16)


# The F16 scratch buffers the tests hand to kDeq / deqW16 (torch memory).
_SENTINELS = []


def sentinel(n):
    t = torch.from_numpy(np.full(n, NAN16, np.uint16).view(np.int16)).cuda()
    _SENTINELS.append(t)
    return t


@pytest.fixture(autouse=True)
def _retire_records():
    """After each test, drop the deferred-dequantisation records on its F16
    scratch buffers (madi_q8_forget over each whole buffer: the records are
    dropped, nothing is written), as a host does before its allocator hands
    the memory to other code.  A record left on freed torch memory would be
    written out into whatever a later test allocates there once that test's
    writes overlap it."""
    yield
    if _SENTINELS:
        import madi_amd.q8 as q8
        for t in _SENTINELS:
            q8.forget(t)
        _SENTINELS.clear()


def normwise(c, ref):
    c = np.asarray(c, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.max(np.abs(c - ref)) / max(np.max(np.abs(ref)), 1e-30)


ROWS = np.unique(np.r_[np.arange(0, M, 32), np.arange(31, M, 32), M - 1])


def check_gemm(c16, a, qs, sc, bias=None, epi=O.EPI_NONE):
    c = host_f16(c16)[ROWS].astype(np.float64)
    ref = O.q8_gemm_rows(a, qs, sc, rows=ROWS, bias=bias, epilogue=epi, threads=16)
    assert np.all(np.isfinite(c))
    err = normwise(c, ref)
    assert err <= TOL, err


def test_encoder_layer_unchanged_sequence(q):
    """One encoder layer's Q8 calls exactly as encoder.zig:262-301 issues them
    on the tensor-op path (K.m4_bias, K.m4_nn, K.m4_bias_gelu all resolved):
    q, k, v with bias from slices of the stacked q|k|v weight through s.wdq
    and s.wdq2, out-proj, fc1 + bias + GELU, and fc2 on fc1's output.  The
    attention and layer-norm kernels between them are not part of this path:
    their outputs are synthetic here."""
    say("encoder layer, unchanged call sequence")
    rng = np.random.default_rng(262)
    m4 = q.getFunction("m4_gemm_nn")
    m4b = q.getFunction("m4_gemm_bias")
    m4bg = q.getFunction("m4_gemm_bias_gelu")
    qkv_qs, qkv_sc = synth.q8_weight(rng, 3 * D, D)
    o_qs, o_sc = synth.q8_weight(rng, D, D)
    m0_qs, m0_sc = synth.q8_weight(rng, MLP, D)
    m2_qs, m2_sc = synth.q8_weight(rng, D, MLP)
    qkv_w, o_w = q.upload_q8(qkv_qs, qkv_sc), q.upload_q8(o_qs, o_sc)
    m0_w, m2_w = q.upload_q8(m0_qs, m0_sc), q.upload_q8(m2_qs, m2_sc)
    q_b, k_b, v_b = (rng.standard_normal(D).astype(np.float32) for _ in range(3))
    m0_b = rng.standard_normal(MLP).astype(np.float32)
    x_ln = synth.activations(rng, M, D)     # layer norm output (kLN)
    ao = synth.activations(rng, M, D)       # attention output (kFlash)
    x_ln2 = synth.activations(rng, M, D)    # bias + residual + layer norm output (kBRLN)
    wdq, wdq2 = sentinel(D * MLP), sentinel(D * MLP)   # Scratch.wdq / wdq2
    d_x, d_ao, d_x2 = dev_f16(x_ln), dev_f16(ao), dev_f16(x_ln2)
    qo, ko, vo, mo = (torch.empty((M, D), dtype=torch.int16, device="cuda") for _ in range(4))
    mh = torch.empty((M, MLP), dtype=torch.int16, device="cuda")
    mo2 = torch.empty((M, D), dtype=torch.int16, device="cuda")
    d_qb, d_kb, d_vb, d_m0b = dev(q_b), dev(k_b), dev(v_b), dev(m0_b)

    # encoder.zig:262-301, the K.m4_bias / K.m4_nn / K.m4_bias_gelu branches
    q.kDeq(wdq, qkv_w, D, D)
    q.kM4Bias(m4b, d_x, wdq, qo, d_qb, M, D, D)
    q.kDeq(wdq2, qkv_w.rows(D, D), D, D)
    q.kM4Bias(m4b, d_x, wdq2, ko, d_kb, M, D, D)
    q.kDeq(wdq, qkv_w.rows(2 * D, D), D, D)
    q.kM4Bias(m4b, d_x, wdq, vo, d_vb, M, D, D)
    q.kDeq(wdq, o_w, D, D)
    q.kM4(m4, d_ao, wdq, mo, M, D, D)
    q.kDeq(wdq, m0_w, MLP, D)
    q.kM4Bias(m4bg, d_x2, wdq, mh, d_m0b, M, MLP, D)
    q.kDeq(wdq2, m2_w, D, MLP)
    q.kM4(m4, mh, wdq2, mo2, M, D, MLP)
    q.sync()

    # the F16 scratch was never written: every product ran the fused Q8 GEMM
    assert np.all(wdq.cpu().numpy().view(np.uint16) == NAN16)
    assert np.all(wdq2.cpu().numpy().view(np.uint16) == NAN16)
    check_gemm(qo, x_ln, qkv_qs[:D], qkv_sc[:D], q_b, O.EPI_BIAS)
    check_gemm(ko, x_ln, qkv_qs[D:2 * D], qkv_sc[D:2 * D], k_b, O.EPI_BIAS)
    check_gemm(vo, x_ln, qkv_qs[2 * D:], qkv_sc[2 * D:], v_b, O.EPI_BIAS)
    check_gemm(mo, ao, o_qs, o_sc)
    check_gemm(mh, x_ln2, m0_qs, m0_sc, m0_b, O.EPI_BIAS_GELU)
    check_gemm(mo2, host_f16(mh), m2_qs, m2_sc)   # fc2 consumes the GPU's fc1 output

    # anything that reads the scratch now sees the dequantised weights: the
    # last kDeq into each buffer (fc1 -> wdq, fc2 -> wdq2), bit for bit
    q.materialize(None)
    q.sync()
    assert np.array_equal(wdq.cpu().numpy().view(np.uint16),
                          O.dequant_q8_f16(m0_qs, m0_sc).view(np.uint16).reshape(-1))
    assert np.array_equal(wdq2.cpu().numpy().view(np.uint16),
                          O.dequant_q8_f16(m2_qs, m2_sc).view(np.uint16).reshape(-1))


def test_encoder_sequence_without_deferral(q):
    """The same pairs with the deferral off: kDeq writes the F16 scratch and
    kM4 / kM4Bias run the library F16 GEMM with the reference's rounding
    order (product rounded to f16, then bias).  Same results to the gate."""
    say("encoder pairs, deferral off")
    rng = np.random.default_rng(263)
    m = 257
    qs, sc = synth.q8_weight(rng, MLP, D)
    w = q.upload_q8(qs, sc)
    bias = rng.standard_normal(MLP).astype(np.float32)
    a = synth.activations(rng, m, D)
    wdq = sentinel(D * MLP)
    c = torch.empty((m, MLP), dtype=torch.int16, device="cuda")
    q.set_deferred_dequant(False)
    try:
        q.kDeq(wdq, w, MLP, D)
        q.kM4Bias("m4_gemm_bias_gelu", dev_f16(a), wdq, c, dev(bias), m, MLP, D)
        q.sync()
    finally:
        q.set_deferred_dequant(True)
    assert np.array_equal(wdq.cpu().numpy().view(np.uint16),
                          O.dequant_q8_f16(qs, sc).view(np.uint16).reshape(-1))
    got = host_f16(c).astype(np.float64)
    ref = O.q8_gemm_rows(a, qs, sc, bias=bias, epilogue=O.EPI_BIAS_GELU, threads=16)
    assert normwise(got, ref) <= TOL


def test_decoder_handles_and_proj(q):
    """decoder.zig: kGemvQ8BiasEpi with the handles of gemv_q8_bias_gelu and
    gemv_q8_bias_res gives the dedicated entry points' results bit for bit;
    proj on deqW16's F16 copies (decoder.zig:337-341) runs the batched
    projection from the Q8 weight (equal to pproj, copies never written), and
    on a true F16 weight the library GEMM (to the gate)."""
    say("decoder handles and proj")
    rng = np.random.default_rng(337)
    qs, sc = synth.q8_weight(rng, MLP, D)
    w = q.upload_q8(qs, sc)
    x = dev(rng.standard_normal(D).astype(np.float32))
    bias = dev(rng.standard_normal(MLP).astype(np.float32))
    res0 = rng.standard_normal(MLP).astype(np.float32)
    for name, direct in (("gemv_q8_bias_gelu", "madi_q8_gemv_bias_gelu"),
                         ("gemv_q8_bias_res", "madi_q8_gemv_bias_res")):
        o1, o2 = dev(res0.copy()), dev(res0.copy())
        q.kGemvQ8BiasEpi(q.getFunction(name), o1, x, w, bias, MLP, D)
        _lib.call(direct, o2.data_ptr(), x.data_ptr(), w.qs, w.scales, bias.data_ptr(), MLP, D)
        q.sync()
        assert torch.equal(o1, o2), name

    B = 8
    wf16 = sentinel(D * MLP)                  # WF16.m0w, [D][MLP]
    in16 = torch.empty(B * MLP, dtype=torch.int16, device="cuda")   # BScratch.in16
    xin = rng.standard_normal((B, D)).astype(np.float32)
    q.deqW16(wf16, w, MLP, D)
    out = torch.empty((B, MLP), dtype=torch.float32, device="cuda")
    q.proj(in16, dev(xin), wf16, out, B, MLP, D)
    want = torch.empty((B, MLP), dtype=torch.float32, device="cuda")
    q.pproj(dev(xin), w, want, B, MLP, D)
    q.sync()
    assert torch.equal(out, want)
    assert np.all(wf16.cpu().numpy().view(np.uint16) == NAN16)
    # a true F16 weight (not recorded): f16 staging + library GEMM, f32 out
    w16 = dev_f16(O.dequant_q8_f16(qs, sc))
    out2 = torch.empty((B, MLP), dtype=torch.float32, device="cuda")
    q.proj(in16, dev(xin), w16, out2, B, MLP, D)
    q.sync()
    assert normwise(out2.cpu().numpy(), O.q8_proj(xin, qs, sc, threads=8)) <= TOL


class DevBuf:
    """A madi_alloc buffer (the library sees its extent)."""

    def __init__(self, nbytes):
        self.n = nbytes
        self.p = _lib.lib().madi_alloc(nbytes)
        assert self.p

    def up(self, arr):
        arr = np.ascontiguousarray(arr)
        _lib.call("madi_upload", self.p, arr.ctypes.data, arr.nbytes)

    def down(self, dtype, count):
        out = np.empty(count, dtype)
        _lib.call("madi_download", out.ctypes.data, self.p, out.nbytes)
        return out

    def free(self):
        _lib.lib().madi_free(self.p)
        self.p = None


def q8_devbufs(q, qs, sc):
    tq, ts = q.repack_host(qs, sc)
    bq, bs = DevBuf(tq.nbytes), DevBuf(ts.nbytes)
    bq.up(tq)
    bs.up(ts)
    return bq, bs


def test_deferred_dequant_is_written_when_observable(q):
    """A recorded kDeq is carried out before anything could see the
    difference: a download of wdq, an upload into the Q8 source, a madi_free
    of the source, a partial overwrite of wdq; a full overwrite drops it."""
    say("deferred dequantisation triggers")
    rng = np.random.default_rng(429)
    n, k = 96, 256
    qs, sc = synth.q8_weight(rng, n, k)
    qs2, sc2 = synth.q8_weight(rng, n, k)
    want = O.dequant_q8_f16(qs, sc).view(np.uint16).reshape(-1)
    nw = n * k
    wdq = DevBuf(nw * 2)
    bq, bs = q8_devbufs(q, qs, sc)

    def fresh_sentinel():
        wdq.up(np.full(nw, NAN16, np.uint16))

    # 1. download of wdq
    fresh_sentinel()
    _lib.call("madi_q8_dequant_f16", wdq.p, bq.p, bs.p, n, k)
    assert np.array_equal(wdq.down(np.uint16, nw), want)
    # 2. an upload into the Q8 source: wdq keeps the weights it was made from
    fresh_sentinel()
    _lib.call("madi_q8_dequant_f16", wdq.p, bq.p, bs.p, n, k)
    tq2, ts2 = q.repack_host(qs2, sc2)
    bq.up(tq2)
    bs.up(ts2)
    assert np.array_equal(wdq.down(np.uint16, nw), want)
    # 3. madi_free of the source
    fresh_sentinel()
    bq.up(q.repack_host(qs, sc)[0])
    bs.up(q.repack_host(qs, sc)[1])
    _lib.call("madi_q8_dequant_f16", wdq.p, bq.p, bs.p, n, k)
    bq.free()
    bs.free()
    assert np.array_equal(wdq.down(np.uint16, nw), want)
    # 4. a partial overwrite of wdq lands on top of the dequantised weights
    bq, bs = q8_devbufs(q, qs, sc)
    fresh_sentinel()
    _lib.call("madi_q8_dequant_f16", wdq.p, bq.p, bs.p, n, k)
    head = np.arange(8, dtype=np.uint16)
    wdq.up(head)
    got = wdq.down(np.uint16, nw)
    assert np.array_equal(got[:8], head) and np.array_equal(got[8:], want[8:])
    # 5. a full overwrite drops the record: a GEMM on wdq multiplies the new data
    _lib.call("madi_q8_dequant_f16", wdq.p, bq.p, bs.p, n, k)
    w16 = (rng.standard_normal((k, n)) * 0.01).astype(np.float16)
    wdq.up(w16.view(np.uint16))
    a = synth.activations(rng, 40, k)
    c = torch.empty((40, n), dtype=torch.int16, device="cuda")
    q.kM4("m4_gemm_nn", dev_f16(a), wdq.p, c, 40, n, k)
    q.sync()
    ref = a.astype(np.float64) @ w16.astype(np.float64)
    assert normwise(host_f16(c), ref) <= TOL
    for b in (wdq, bq, bs):
        b.free()


VOCAB = 51866


@pytest.fixture(scope="module")
def tok_emb(q):
    """The tied token embedding as a Q8 weight [VOCAB][D] (seeded, synthetic)."""
    rng = np.random.default_rng(2391)
    qs, sc = synth.q8_weight(rng, VOCAB, D)
    return qs, sc, q.upload_q8(qs, sc)


def test_batched_logits_unchanged_sequence(q, tok_emb):
    """The batched decode's logit step exactly as transcribe.zig:1358 and
    2391-2394 issue it: deqW16 of the tied tok_emb into bb_temb once, then per
    step kCvt32 (f32 -> f16 rows), matmulF16Batched(bb_x16, bb_temb, bb_l16,
    B, VOCAB, D) and kCvt16.  The two conversions are engine kernels outside
    this path (torch casts here).  bb_temb is never written (the product ran
    from the Q8 weight, 51866 rows with a 26-row last panel); the f16 logits
    equal the batched projection's f32 sums rounded once to f16, bit for bit
    (same kernel, same accumulation order), and match the oracle."""
    qs, sc, w = tok_emb
    bb_temb = sentinel(D * VOCAB)
    q.deqW16(bb_temb, w, VOCAB, D)
    rng = np.random.default_rng(2393)
    for B in (8, 16, 3):
        say(f"batched logits B={B}")
        xb = rng.standard_normal((B, D)).astype(np.float32)
        bb_x16 = dev(xb).half().view(torch.int16)                        # kCvt32
        bb_l16 = sentinel(B * VOCAB)
        q.matmulF16Batched(bb_x16, bb_temb, bb_l16, B, VOCAB, D)
        logits = bb_l16.view(torch.float16).float()                      # kCvt16
        want = torch.empty((B, VOCAB), dtype=torch.float32, device="cuda")
        q.pproj(bb_x16.view(torch.float16).float(), w, want, B, VOCAB, D)
        q.sync()
        assert torch.equal(bb_l16.view(torch.float16).view(B, VOCAB), want.half()), B
        x16 = host_f16(bb_x16).reshape(B, D)
        ref = O.q8_gemm_rows(x16, qs, sc, threads=16)
        got = logits.cpu().numpy().reshape(B, VOCAB)
        assert np.all(np.isfinite(got))
        assert normwise(got, ref) <= TOL, B
    assert np.all(bb_temb.cpu().numpy().view(np.uint16) == NAN16)


def test_cross_kv_unchanged_sequence(q):
    """The per-slot cross-attention K/V build exactly as transcribe.zig:
    2440-2448 issues it: per layer deqW16(cross_wdq, ckw) then
    matmulF16Batched(eo16, cross_wdq, ckc, actx, D, D), and the same for V
    (biasAdd16 after it is an engine kernel outside this path).  actx is the
    full window (1500 rows, fused GEMM), a shrunk audio context (750, fused
    GEMM) and a short one (100, the batched projection kernel).  cross_wdq is
    never written; K and V match the oracle; rows past actx of the ENC_SEQ-row
    caches are untouched."""
    rng = np.random.default_rng(2440)
    ckq, cks = synth.q8_weight(rng, D, D)
    cvq, cvs = synth.q8_weight(rng, D, D)
    ckw, cvw = q.upload_q8(ckq, cks), q.upload_q8(cvq, cvs)
    eo = synth.activations(rng, M, D)
    eo16 = dev_f16(eo)
    cross_wdq = sentinel(D * D)
    for actx in (1500, 750, 100):
        say(f"cross K/V actx={actx}")
        ckc, cvc = sentinel(M * D), sentinel(M * D)
        q.deqW16(cross_wdq, ckw, D, D)
        q.matmulF16Batched(eo16, cross_wdq, ckc, actx, D, D)
        q.deqW16(cross_wdq, cvw, D, D)
        q.matmulF16Batched(eo16, cross_wdq, cvc, actx, D, D)
        q.sync()
        assert np.all(cross_wdq.cpu().numpy().view(np.uint16) == NAN16)
        rows = ROWS[ROWS < actx]
        for cache, wq, ws in ((ckc, ckq, cks), (cvc, cvq, cvs)):
            h = cache.cpu().numpy().view(np.uint16).reshape(M, D)
            assert np.all(h[actx:] == NAN16), actx
            got = h[rows].view(np.float16).astype(np.float64)
            assert np.all(np.isfinite(got))
            ref = O.q8_gemm_rows(eo[:actx], wq, ws, rows=rows, threads=16)
            assert normwise(got, ref) <= TOL, actx


def test_matmul_f16_recorded_any_width(q):
    """matmulF16Batched on a recorded copy whose width is not a multiple of 32
    or even of 2 (97 and 1002 rows: partial last panels, 2- and 4-byte aligned
    output rows) runs the batched projection kernel; alpha / beta other than
    (1, 0) materialise the copy and run the library GEMM on it."""
    rng = np.random.default_rng(4242)
    k = 256
    for n, m in ((97, 5), (1002, 24), (97, 40)):
        say(f"recorded copy n={n} m={m}")
        qs, sc = synth.q8_weight(rng, n, k)
        w = q.upload_q8(qs, sc)
        wdq = sentinel(k * n)
        q.deqW16(wdq, w, n, k)
        a = synth.activations(rng, m, k)
        c = sentinel(m * n)
        q.matmulF16Batched(dev_f16(a), wdq, c, m, n, k)
        q.sync()
        assert np.all(wdq.cpu().numpy().view(np.uint16) == NAN16)
        got = host_f16(c).reshape(m, n).astype(np.float64)
        assert normwise(got, O.q8_gemm_rows(a, qs, sc)) <= TOL
        # alpha = 0.5: the library GEMM on the materialised copy
        c2 = sentinel(m * n)
        q.matmulF16Batched(dev_f16(a), wdq, c2, m, n, k, alpha=0.5)
        q.sync()
        assert np.array_equal(wdq.cpu().numpy().view(np.uint16),
                              O.dequant_q8_f16(qs, sc).view(np.uint16).reshape(-1))
        got2 = host_f16(c2).reshape(m, n).astype(np.float64)
        assert normwise(got2, 0.5 * O.q8_gemm_rows(a, qs, sc)) <= TOL


def test_outside_writes_announced_with_forget(q):
    """Writes by code outside the library (torch copies here) into a recorded
    wdq or its Q8 source, announced with madi_q8_forget: a full overwrite of
    wdq drops the record (the next F16 GEMM multiplies the new data), a
    partial one lands on top of the dequantised weights, and a write into the
    Q8 source leaves wdq with the weights it was recorded from."""
    say("outside writes and madi_q8_forget")
    rng = np.random.default_rng(4388)
    n, k, m = 128, 256, 40
    qs, sc = synth.q8_weight(rng, n, k)
    want = O.dequant_q8_f16(qs, sc).view(np.uint16).reshape(-1)
    w = q.upload_q8(qs, sc)
    a = synth.activations(rng, m, k)
    # 1. full overwrite of wdq from torch
    wdq = sentinel(k * n)
    q.kDeq(wdq, w, n, k)
    w16 = (rng.standard_normal((k, n)) * 0.01).astype(np.float16)
    q.forget(wdq)
    wdq.copy_(dev_f16(w16).view(-1))
    c = torch.empty((m, n), dtype=torch.int16, device="cuda")
    q.kM4("m4_gemm_nn", dev_f16(a), wdq, c, m, n, k)
    q.sync()
    ref = a.astype(np.float64) @ w16.astype(np.float64)
    assert normwise(host_f16(c), ref) <= TOL
    # 2. partial overwrite of the head: the record shrinks to the rest, which
    # a reader outside the library gets with madi_q8_materialize (the head
    # written from torch is left alone)
    wdq = sentinel(k * n)
    q.kDeq(wdq, w, n, k)
    head = wdq[:64]
    q.forget(head)
    head.copy_(torch.arange(64, dtype=torch.int16, device="cuda"))
    q.materialize(wdq)
    q.sync()
    got = wdq.cpu().numpy().view(np.uint16)
    assert np.array_equal(got[:64], np.arange(64, dtype=np.uint16))
    assert np.array_equal(got[64:], want[64:])
    # 3. a write into the Q8 source: wdq keeps the recorded weights
    wdq = sentinel(k * n)
    src = q.upload_q8(qs, sc)
    q.kDeq(wdq, src, n, k)
    qt = src._keep[0]
    q.forget(qt)
    qt.zero_()
    q.sync()
    assert np.array_equal(wdq.cpu().numpy().view(np.uint16), want)


def test_issue_list_replays_the_engine_layer(q):
    """The encoder layer of test_encoder_layer_unchanged_sequence recorded in
    an IssueList and replayed from C (the bench's issue path) gives the same
    bits as the calls made one by one from Python."""
    say("issue list replay of one encoder layer")
    from madi_amd.issue import IssueList
    rng = np.random.default_rng(2626)
    m = 700
    qkv_w = q.upload_q8(*synth.q8_weight(rng, 3 * D, D))
    m0_w = q.upload_q8(*synth.q8_weight(rng, MLP, D))
    m2_w = q.upload_q8(*synth.q8_weight(rng, D, MLP))
    qb, m0b = dev(rng.standard_normal(D).astype(np.float32)), dev(rng.standard_normal(MLP).astype(np.float32))
    x = dev_f16(synth.activations(rng, m, D))
    wdq, wdq2 = sentinel(D * MLP), sentinel(D * MLP)
    outs = []
    for how in ("python", "c"):
        qo = torch.empty((m, D), dtype=torch.int16, device="cuda")
        ko = torch.empty((m, D), dtype=torch.int16, device="cuda")
        mh = torch.empty((m, MLP), dtype=torch.int16, device="cuda")
        mo = torch.empty((m, D), dtype=torch.int16, device="cuda")
        lst = IssueList() if how == "c" else q
        lst.kDeq(wdq, qkv_w, D, D)
        lst.kM4Bias(q.getFunction("m4_gemm_bias"), x, wdq, qo, qb, m, D, D)
        lst.kDeq(wdq2, qkv_w.rows(D, D), D, D)
        lst.kM4Bias(q.getFunction("m4_gemm_bias"), x, wdq2, ko, qb, m, D, D)
        lst.kDeq(wdq, m0_w, MLP, D)
        lst.kM4Bias(q.getFunction("m4_gemm_bias_gelu"), x, wdq, mh, m0b, m, MLP, D)
        lst.kDeq(wdq2, m2_w, D, MLP)
        lst.kM4(q.getFunction("m4_gemm_nn"), mh, wdq2, mo, m, D, MLP)
        if how == "c":
            lst.run(2)
        q.sync()
        outs.append([t.cpu().numpy() for t in (qo, ko, mh, mo)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    assert np.all(wdq.cpu().numpy().view(np.uint16) == NAN16)


def test_smaller_kdeq_shortens_the_earlier_record(q):
    """The encoder's scratch pattern: kDeq of fc1 (5120 x 1280) into wdq, then
    the next layer's kDeq of q (1280 x 1280) into the start of the same
    buffer.  The second record takes the head; the first keeps the rest
    without writing it (the fused GEMM on the second still runs and wdq stays
    a sentinel), and whatever reads wdq later sees exactly what the two kDeq
    calls would have left there: q's weights, then the tail of fc1's."""
    say("smaller kDeq over an earlier record")
    rng = np.random.default_rng(297)
    big_q, big_s = synth.q8_weight(rng, MLP, D)
    sm_q, sm_s = synth.q8_weight(rng, D, D)
    big, sm = q.upload_q8(big_q, big_s), q.upload_q8(sm_q, sm_s)
    wdq = sentinel(D * MLP)
    m = 64
    a = synth.activations(rng, m, D)
    c = torch.empty((m, D), dtype=torch.int16, device="cuda")
    q.kDeq(wdq, big, MLP, D)
    q.kDeq(wdq, sm, D, D)
    q.kM4("m4_gemm_nn", dev_f16(a), wdq, c, m, D, D)
    q.sync()
    assert np.all(wdq.cpu().numpy().view(np.uint16) == NAN16)
    assert normwise(host_f16(c).astype(np.float64), O.q8_gemm_rows(a, sm_q, sm_s)) <= TOL
    q.materialize(wdq)
    q.sync()
    got = wdq.cpu().numpy().view(np.uint16)
    head = O.dequant_q8_f16(sm_q, sm_s).view(np.uint16).reshape(-1)
    tail = O.dequant_q8_f16(big_q, big_s).view(np.uint16).reshape(-1)
    assert np.array_equal(got[:D * D], head)
    assert np.array_equal(got[D * D:], tail[D * D:])
    # a write strictly inside an owed range splits it: the weights are written
    # out at once and the write lands on top
    wdq2 = DevBuf(D * D * 2)
    _lib.call("madi_q8_dequant_f16", wdq2.p, sm.qs, sm.scales, D, D)
    mid = np.full(16, 7, np.uint16)
    _lib.call("madi_upload", wdq2.p + 4096, mid.ctypes.data, mid.nbytes)
    got2 = wdq2.down(np.uint16, D * D)
    want2 = head.copy()
    want2[2048:2064] = 7
    assert np.array_equal(got2, want2)
    wdq2.free()


def test_qkv_slices_run_as_one_grouped_launch(q):
    """encoder.zig:262-267 with the stacked q|k|v weight in its own madi_alloc
    allocation (as the engine's loader makes it): the q GEMM is held (its
    output untouched after the call), k joins, and v completes the group,
    which runs as one stacked 1280 -> 3840 launch into the three blocks of
    s.qkv.  The outputs equal, bit for bit, the three GEMMs launched one by
    one (grouping off: the same MFMA order per output), and the oracle.  A
    held group is launched by madi_sync, by a library read of a held output,
    by a write of a held operand, and by a GEMM that does not join."""
    say("q|k|v grouping")
    rng = np.random.default_rng(267)
    m = 1500
    qkv_qs, qkv_sc = synth.q8_weight(rng, 3 * D, D)
    w = q.upload_q8_alloc(qkv_qs, qkv_sc)
    b = [dev(rng.standard_normal(D).astype(np.float32)) for _ in range(3)]
    x = synth.activations(rng, m, D)
    d_x = dev_f16(x)
    wdq, wdq2 = sentinel(D * D), sentinel(D * D)
    m4b = q.getFunction("m4_gemm_bias")

    def issue(qkv, upto=3):
        q.kDeq(wdq, w, D, D)
        q.kM4Bias(m4b, d_x, wdq, qkv[0], b[0], m, D, D)
        if upto > 1:
            q.kDeq(wdq2, w.rows(D, D), D, D)
            q.kM4Bias(m4b, d_x, wdq2, qkv[1], b[1], m, D, D)
        if upto > 2:
            q.kDeq(wdq, w.rows(2 * D, D), D, D)
            q.kM4Bias(m4b, d_x, wdq, qkv[2], b[2], m, D, D)

    grouped = sentinel(3 * m * D).view(3, m, D)
    q.set_gemm_grouping(True)
    # held: after the q call (and a device-wide wait outside the library) the
    # q block is still the sentinel
    issue(grouped, upto=1)
    torch.cuda.synchronize()
    assert np.all(grouped[0].cpu().numpy().view(np.uint16) == NAN16)
    issue(grouped, upto=3)   # q again (replaces nothing: joins are by slice), k, v
    q.sync()
    g = grouped.cpu().numpy().view(np.uint16)
    q.set_gemm_grouping(False)
    single = sentinel(3 * m * D).view(3, m, D)
    issue(single)
    q.sync()
    q.set_gemm_grouping(True)
    s_ = single.cpu().numpy().view(np.uint16)
    assert np.array_equal(g, s_)
    for i in range(3):
        check_gemm(grouped[i], x, qkv_qs[i * D:(i + 1) * D], qkv_sc[i * D:(i + 1) * D],
                   b[i].cpu().numpy(), O.EPI_BIAS)
    assert np.all(wdq.cpu().numpy().view(np.uint16) == NAN16)

    # what launches a held group
    def held_then(action, upto=1):
        out = sentinel(3 * m * D).view(3, m, D)
        issue(out, upto=upto)
        action(out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint16)
        assert np.array_equal(got[:upto], s_[:upto]), action
        q.sync()
    held_then(lambda out: q.sync())
    held_then(lambda out: _lib.call("madi_download", np.empty(8, np.uint16).ctypes.data,
                                    out[1].data_ptr(), 16), upto=2)      # a read of k
    o_qs, o_sc = synth.q8_weight(rng, D, D)
    o_w = q.upload_q8(o_qs, o_sc)
    mo = sentinel(m * D)

    def out_proj(out):  # the next kDeq + kM4 pair (out-proj): does not join
        q.kDeq(wdq, o_w, D, D)
        q.kM4("m4_gemm_nn", d_x, wdq, mo, m, D, D)
    held_then(out_proj, upto=2)
    held_then(lambda out: _lib.call("madi_upload", d_x.data_ptr(),
                                    np.ascontiguousarray(x[:4]).ctypes.data, 16))  # a write of x
