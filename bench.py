"""Benchmark of the MI355X Q8 matmul path (one GPU).

A step is one pass of the hot path over one batch of synthetic input:
  1. the encoder fc1 Q8 GEMM, A f16 [1500, 1280] x W int8 [5120, 1280] (+ fp16
     per-32 scales) -> C f16 [1500, 5120], fp32 accumulation;
  2. the decoder vocab-logit Q8 GEMV with f32 activations, as the engine
     calls it (kLogitGemv, madi_q8_logit_gemv): x f32 [1280] x W int8
     [51866, 1280] -> f32 logits [51866], cold: the step cycles through 4
     distinct weight copies (4 x 70.75 MB > the 256 MB Infinity Cache) so
     each launch streams HBM;
  3. the same vocab GEMV with fp16 activations, on the same rotation.
Inputs are resident in HBM before the timed region.  The timed region runs
the K steps' GEMMs back to back, then their f32-activation GEMVs, then their
fp16-activation GEMVs, with HIP events on the kernels' stream at the start,
between the runs and at the end, so each kernel's average duration is
(event span) / K -- the figure rocprofv3's
kernel trace reports for the same launches (a per-launch event pair would add
the dispatch gap).  The JSON line reports the GEMM as the headline value
(TFLOP/s) and the GEMV beside it (GB/s), each with its roofline fraction and,
when profiles/traffic_q8_fc1_gemm_vocab_gemv.md holds them, the measured HBM
bytes per launch, plus the restated reference CPU path timed on this host's
cores (a reported baseline only).

Beside the headline, "configs" reports the other measured workloads, each
call sequence issued from compiled code (madi_amd.issue, a C loop over the
library's calls, as the engine issues from Zig): the encoder GEMM set of one
30 s window (32 layers, independent weights) with q|k|v stacked, and the same
window as the engine's layer loop issues it (q, k, v through kDeq + kM4Bias on
slices of the stacked weight, grouped into one launch at the boundary) and in
its F16-cache mode (kM4 / kM4Bias on true F16 weights through the NN f16
GEMM), a batched decode step at M = 8 and 16 (skinny Q8 projections, cold weights) with
the per-chunk cross-attention K|V GEMM, one decoder token at M = 1 through the
GEMV family (and its fused q|k|v GEMV alone), one decoder layer's sequence
prefill projections at M = 320, the 16-window long-audio fc1/fc2, and the
encoder self-attention of one window over its Q/K/V projections.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-configs]
       python bench.py --config NAME     (one configuration alone, e.g. encoder_attention)
       python bench.py --calibrate-copy   (a plain 256 MiB device copy, the
                                           reference kernel for FETCH_SIZE /
                                           WRITE_SIZE scaling)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2516.6   # MI355X dense fp16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

M, K, N = 1500, 1280, 5120          # encoder fc1 at one 30 s window
VOCAB, DIM = 51866, 1280            # decoder vocab logits
GEMV_COPIES = 4
COPY_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_q8_fc1_gemm_vocab_gemv.md")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def gemm_flops():
    return 2.0 * M * N * K


def gemm_bytes():
    return M * K * 2 + N * K + N * (K // 32) * 2 + M * N * 2


def gemv_bytes():
    return VOCAB * DIM + VOCAB * (DIM // 32) * 2 + DIM * 2 + VOCAB * 4


def cpu_share() -> int:
    """Host threads the CPU baseline may use: the CPUs this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (a one-GPU share
    of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def _median_time(fn, runs: int) -> float:
    fn()  # warm-up
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return float(np.median(ts))


def cpu_baseline(threads: int, runs: int = 5):
    """The oracle (C restatement of the reference's CPU loop,
    engine/metal/test_q8gemm.zig:59-69: dequantise to fp32, k-sequential fp32
    accumulation) built for this host (-O3 -march=native, no BLAS), on the
    same fc1 and vocab workloads: (i) the literal single-thread loop on a
    96-row sample of fc1 (rows are independent: the rate per row is the
    rate) and the full vocab GEMV, (ii) OpenMP over output rows on `threads`
    threads for all 1500 rows and the vocab GEMV; each the median of `runs`
    runs after one warm-up."""
    import tempfile
    import oracle as O
    from madi_amd import synth
    build = "prebuilt -O3 -march=x86-64-v3 (no compiler on this host)"
    native = O.build_native(tempfile.mkdtemp(prefix="madi_oracle_"))
    if native:
        O.use_library(native)
        build = "-O3 -march=native -ffp-contract=off -fopenmp (built here)"
    a, qs, sc = synth.gemm_case(0, M, N, K)
    rows1 = np.arange(0, M, M // 96, dtype=np.uint32)[:96]
    rowsn = np.arange(0, M, dtype=np.uint32)
    f_row = 2.0 * N * K
    dt1 = _median_time(lambda: O.q8_gemm_rows(a, qs, sc, rows=rows1, threads=1), runs)
    dtn = _median_time(lambda: O.q8_gemm_rows(a, qs, sc, rows=rowsn, threads=threads), runs)
    x, qv, sv = synth.gemv_case(0, VOCAB, DIM)
    xf = x.astype(np.float32)
    dtv1 = _median_time(lambda: O.q8_gemv(xf, qv, sv, threads=1), runs)
    dtvn = _median_time(lambda: O.q8_gemv(xf, qv, sv, threads=threads), runs)
    return {
        "gemm_1t_tflops": f_row * rows1.size / dt1 / 1e12,
        "gemm_nt_tflops": f_row * rowsn.size / dtn / 1e12,
        "gemv_1t_gbs": gemv_bytes() / dtv1 / 1e9,
        "gemv_nt_gbs": gemv_bytes() / dtvn / 1e9,
        "build": build,
        "sample": (f"fc1 GEMM: {rows1.size} of {M} rows on 1 thread ({dt1:.2f} s per run) and all "
                   f"{rowsn.size} rows on {threads} threads ({dtn:.2f} s); vocab GEMV 1x{DIM}x{VOCAB} "
                   f"in full on 1 ({dtv1:.3f} s) and {threads} threads ({dtvn:.3f} s); median of "
                   f"{runs} runs after a warm-up each"),
    }


# ---------------------------------------------------------------- other configurations
# Encoder projection shapes per layer (large-v3-turbo, d_model 1280, MLP 5120)
ENC_LAYERS, DEC_LAYERS = 32, 4
ENC_SHAPES = [("qkv", 3840, 1280), ("out", 1280, 1280), ("fc1", 5120, 1280), ("fc2", 1280, 5120)]
DEC_SHAPES = [("self_qkv", 3840, 1280), ("self_out", 1280, 1280), ("cross_q", 1280, 1280),
              ("cross_out", 1280, 1280), ("ffn_up", 5120, 1280), ("ffn_down", 1280, 5120)]


def _timed(torch, stream, fn, reps, settle=False):
    """Average seconds per call of fn() over `reps` back-to-back calls, after
    untimed calls with the last min(reps, 8) indices (the first shape of a
    configuration otherwise pays for the clocks ramping up after the set-up's
    copies; the timed calls then start with the weight copy used longest ago,
    as in the steady state of the rotation).  The timed calls follow the
    untimed ones with the GPU still busy, the steady state of the engine's
    loops; with `settle` the host waits for the GPU in between, so the timed
    region starts from an idle GPU and shows the rate at which the caller
    issues (the Python-issued figures)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(max(reps - 8, 0), reps):
        fn(i)
    if settle:
        torch.cuda.synchronize()
    e0.record(stream)
    for i in range(reps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


def _timed_list(torch, stream, lst, reps, per=1):
    """Average seconds per `per` calls' worth of lst (an IssueList replayed from
    C) over `reps` back-to-back replays, after min(reps, 4) untimed ones that
    are still running when the timed replays start."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    lst.run(min(reps, 4))
    e0.record(stream)
    lst.run(reps)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / (reps * per)


def _upload_layer(q8, seed, n, k):
    from madi_amd import synth
    qs, sc = synth.q8_weight(np.random.default_rng(seed), n, k)
    return q8.upload_q8(qs, sc)


def config_encoder_window(torch, stream, q8, reps=3):
    """The encoder GEMM set of one 30 s window: 32 layers x (q|k|v stacked
    1280->3840, out 1280->1280, fc1 1280->5120 + bias + GELU, fc2 5120->1280 +
    bias) at M = 1500, independent seeded weights per layer (668 MB, so every
    layer's weights stream from HBM).  Issued from C (madi_amd.issue)."""
    from madi_amd import synth
    from madi_amd.issue import IssueList
    m = 1500
    a = torch.from_numpy(synth.activations(np.random.default_rng(100), m, 5120).view(np.int16)).cuda()
    c = torch.empty((m, 5120), dtype=torch.int16, device="cuda")
    bias = torch.from_numpy(np.random.default_rng(101).standard_normal(5120).astype(np.float32)).cuda()
    layers = [[_upload_layer(q8, 1000 + 4 * l + j, n, k) for j, (_, n, k) in enumerate(ENC_SHAPES)]
              for l in range(ENC_LAYERS)]
    torch.cuda.synchronize()
    EPI = {0: (None, q8.EPI_NONE), 1: (None, q8.EPI_NONE), 2: (bias, q8.EPI_BIAS_GELU),
           3: (bias, q8.EPI_BIAS)}
    window = IssueList()
    for ws in layers:
        for j, (_, n, k) in enumerate(ENC_SHAPES):
            window.kGemmQ8(a, ws[j], c, m, n, k, *EPI[j])
    t = _timed_list(torch, stream, window, reps)
    flops = ENC_LAYERS * sum(2.0 * m * n * k for _, n, k in ENC_SHAPES)
    per = {}
    for j, (name, n, k) in enumerate(ENC_SHAPES):
        one = IssueList()
        for ws in layers:
            one.kGemmQ8(a, ws[j], c, m, n, k, *EPI[j])
        tj = _timed_list(torch, stream, one, 2, per=ENC_LAYERS)
        per[name] = {"us": round(tj * 1e6, 2), "tflops": round(2.0 * m * n * k / tj / 1e12, 1)}
    del layers
    return {
        "workload": "32 layers x (qkv 1280->3840, out 1280->1280, fc1 1280->5120 +bias+GELU, "
                    "fc2 5120->1280 +bias) Q8 GEMMs at M=1500, independent weights per layer, "
                    "issued from C",
        "ms_per_window": round(t * 1e3, 4), "tflop_per_window": round(flops / 1e12, 4),
        "tflops": round(flops / t / 1e12, 1),
        "frac_fp16_peak": round(flops / t / 1e12 / PEAK_FP16_TFLOPS, 4),
        "per_gemm_cold": per,
    }


def config_encoder_window_engine(torch, stream, q8, reps=3):
    """The encoder's Q8 GEMMs of one 30 s window exactly as encoder.zig:256-303
    issues them on its tensor-op path: per layer kDeq of each Q8 weight into the
    F16 scratch (s.wdq / s.wdq2) and kM4 / kM4Bias through the handles of
    m4_gemm_bias, m4_gemm_nn and m4_gemm_bias_gelu: q, k and v as three
    1280->1280 GEMMs + bias from row slices of the stacked q|k|v weight into
    the three blocks of s.qkv, out-proj 1280->1280 without bias, fc1
    1280->5120 + bias + GELU, fc2 5120->1280 without bias (its bias goes into
    the next layer norm).  32 layers, independent weights (each in its own
    madi_alloc allocation, as the engine's loader makes them), M = 1500,
    issued from C through the boundary (madi_m4_gemm on the recorded
    scratch; the q, k, v calls run as one grouped launch).  Also timed with
    the grouping off (three launches)."""
    from madi_amd import synth
    from madi_amd.issue import IssueList
    m, d, mlp = 1500, DIM, 5120
    rng = np.random.default_rng(110)
    f16 = lambda r, c_: torch.from_numpy(synth.activations(rng, r, c_).view(np.int16)).cuda()
    f32 = lambda n: torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    x_ln, ao, x_ln2 = f16(m, d), f16(m, d), f16(m, d)
    qkv = torch.empty((3, m, d), dtype=torch.int16, device="cuda")   # s.qkv: q | k | v blocks
    mo = torch.empty((m, d), dtype=torch.int16, device="cuda")
    mh = torch.empty((m, mlp), dtype=torch.int16, device="cuda")
    wdq = torch.empty(d * mlp, dtype=torch.int16, device="cuda")     # Scratch.wdq
    wdq2 = torch.empty(d * mlp, dtype=torch.int16, device="cuda")    # Scratch.wdq2
    m4, m4b, m4bg = (q8.getFunction(nm) for nm in ("m4_gemm_nn", "m4_gemm_bias", "m4_gemm_bias_gelu"))
    from madi_amd import synth as _s

    def alloc_layer(seed, n, k):  # each weight in its own madi_alloc allocation, as the loader
        return q8.upload_q8_alloc(*_s.q8_weight(np.random.default_rng(seed), n, k))
    layers = []
    for l in range(ENC_LAYERS):
        layers.append(dict(
            qkv=alloc_layer(6000 + 8 * l, 3 * d, d), o=alloc_layer(6001 + 8 * l, d, d),
            m0=alloc_layer(6002 + 8 * l, mlp, d), m2=alloc_layer(6003 + 8 * l, d, mlp),
            qb=f32(d), kb=f32(d), vb=f32(d), m0b=f32(mlp)))
    torch.cuda.synchronize()
    q_, k_, v_ = (qkv[i] for i in range(3))
    window = IssueList()
    for L in layers:
        window.kDeq(wdq, L["qkv"], d, d)
        window.kM4Bias(m4b, x_ln, wdq, q_, L["qb"], m, d, d)
        window.kDeq(wdq2, L["qkv"].rows(d, d), d, d)
        window.kM4Bias(m4b, x_ln, wdq2, k_, L["kb"], m, d, d)
        window.kDeq(wdq, L["qkv"].rows(2 * d, d), d, d)
        window.kM4Bias(m4b, x_ln, wdq, v_, L["vb"], m, d, d)
        window.kDeq(wdq, L["o"], d, d)
        window.kM4(m4, ao, wdq, mo, m, d, d)
        window.kDeq(wdq, L["m0"], mlp, d)
        window.kM4Bias(m4bg, x_ln2, wdq, mh, L["m0b"], m, mlp, d)
        window.kDeq(wdq2, L["m2"], d, mlp)
        window.kM4(m4, mh, wdq2, mo, m, d, mlp)
    t = _timed_list(torch, stream, window, reps)
    q8.set_gemm_grouping(False)   # q, k, v as three launches, for comparison
    t3 = _timed_list(torch, stream, window, reps)
    q8.set_gemm_grouping(True)
    flops = ENC_LAYERS * 2.0 * m * (4 * d * d + 2 * d * mlp)
    del layers
    return {
        "ungrouped_ms_per_window": round(t3 * 1e3, 4),
        "ungrouped_frac_fp16_peak": round(flops / t3 / 1e12 / PEAK_FP16_TFLOPS, 4),
        "workload": "32 layers x (q, k, v 1280->1280 +bias from slices of the stacked weight, "
                    "out 1280->1280, fc1 1280->5120 +bias+GELU, fc2 5120->1280) at M=1500 as "
                    "encoder.zig:256-303 issues them (kDeq + kM4/kM4Bias handles through the "
                    "deferred dequantisation, q|k|v grouped into one launch), independent "
                    "weights per layer, issued from C",
        "ms_per_window": round(t * 1e3, 4), "tflop_per_window": round(flops / 1e12, 4),
        "tflops": round(flops / t / 1e12, 1),
        "frac_fp16_peak": round(flops / t / 1e12 / PEAK_FP16_TFLOPS, 4),
    }


def config_encoder_window_f16cache(torch, stream, q8, reps=3):
    """The encoder window in the engine's F16-cache mode (ENC_F16_CACHE,
    transcribe.zig:1149): every projection holds a true F16 weight [K][N]
    (L.q_f16 .. L.m2_f16) and encoder.zig:262-301 calls kM4 / kM4Bias on it
    with no kDeq: q, k, v 1280->1280 + bias, out 1280->1280, fc1 1280->5120 +
    bias + GELU, fc2 5120->1280.  32 layers, independent weights (1.26 GB of
    F16), M = 1500, issued from C through madi_m4_gemm (the NN f16 GEMM)."""
    from madi_amd.issue import IssueList
    m, d, mlp = 1500, DIM, 5120
    g = torch.Generator(device="cuda").manual_seed(111)
    f16 = lambda *shape, s=1.0: (torch.randn(shape, generator=g, device="cuda") * s).half()
    x_ln, ao, x_ln2 = f16(m, d), f16(m, d), f16(m, d)
    qkv = torch.empty((3, m, d), dtype=torch.half, device="cuda")
    mo = torch.empty((m, d), dtype=torch.half, device="cuda")
    mh = torch.empty((m, mlp), dtype=torch.half, device="cuda")
    m4, m4b, m4bg = (q8.getFunction(nm) for nm in ("m4_gemm_nn", "m4_gemm_bias", "m4_gemm_bias_gelu"))
    layers = []
    for _ in range(ENC_LAYERS):
        layers.append(dict(q=f16(d, d, s=0.03), k=f16(d, d, s=0.03), v=f16(d, d, s=0.03),
                           o=f16(d, d, s=0.03), m0=f16(d, mlp, s=0.03), m2=f16(mlp, d, s=0.015),
                           qb=torch.randn(d, generator=g, device="cuda"),
                           kb=torch.randn(d, generator=g, device="cuda"),
                           vb=torch.randn(d, generator=g, device="cuda"),
                           m0b=torch.randn(mlp, generator=g, device="cuda")))
    torch.cuda.synchronize()
    window = IssueList()
    for L in layers:
        for w, bias_, out in ((L["q"], L["qb"], qkv[0]), (L["k"], L["kb"], qkv[1]), (L["v"], L["vb"], qkv[2])):
            window.kM4Bias(m4b, x_ln, w, out, bias_, m, d, d)
        window.kM4(m4, ao, L["o"], mo, m, d, d)
        window.kM4Bias(m4bg, x_ln2, L["m0"], mh, L["m0b"], m, mlp, d)
        window.kM4(m4, mh, L["m2"], mo, m, d, mlp)
    t = _timed_list(torch, stream, window, reps)
    flops = ENC_LAYERS * 2.0 * m * (4 * d * d + 2 * d * mlp)
    del layers
    return {
        "workload": "32 layers x (q, k, v 1280->1280 +bias, out 1280->1280, fc1 1280->5120 "
                    "+bias+GELU, fc2 5120->1280) at M=1500 on true F16 weights [K][N], as "
                    "encoder.zig:262-301 issues them in the F16-cache mode (kM4 / kM4Bias, no "
                    "kDeq), independent weights per layer, issued from C",
        "ms_per_window": round(t * 1e3, 4), "tflop_per_window": round(flops / 1e12, 4),
        "tflops": round(flops / t / 1e12, 1),
        "frac_fp16_peak": round(flops / t / 1e12 / PEAK_FP16_TFLOPS, 4),
    }


def config_batched_decode(torch, stream, q8, reps=20):
    """One batched decode step at M = 8 and 16 token rows: 4 decoder layers x
    (self q|k|v 1280->3840, self out, cross q, cross out 1280->1280, FFN
    1280->5120->1280) through the skinny Q8 projection (f32 rows, as proj
    reaches it), then the vocab logits 1280->51866 as the engine issues them
    (transcribe.zig:2391-2394: matmulF16Batched on deqW16's recorded copy of
    the tied tok_emb, f16 rows in and out), two alternating weight sets
    (2 x 168 MB > the 256 MB Infinity Cache); plus the per-chunk
    cross-attention K|V projection 1280->2560 at M = 1500 (GEMM)."""
    from madi_amd import synth
    sets = []
    for s_ in range(2):
        layers = [[_upload_layer(q8, 2000 + 100 * s_ + 8 * l + j, n, k)
                   for j, (_, n, k) in enumerate(DEC_SHAPES)] for l in range(DEC_LAYERS)]
        vocab = _upload_layer(q8, 2900 + s_, VOCAB, DIM)
        sets.append((layers, vocab))
    xin = torch.from_numpy(np.random.default_rng(102).standard_normal((16, 5120)).astype(np.float32)).cuda()
    out = torch.empty((16, VOCAB), dtype=torch.float32, device="cuda")
    # the logit step's operands: the f16 rows (bb_x16), deqW16's copy of each
    # set's tok_emb (recorded, never written: the Q8 weight is what is read)
    # and the f16 logits (bb_l16)
    x16 = xin[:, :DIM].contiguous().half().view(torch.int16)
    l16 = torch.empty((16, VOCAB), dtype=torch.int16, device="cuda")
    temb = [torch.empty(VOCAB * DIM, dtype=torch.int16, device="cuda") for _ in sets]
    for t16, (_, vocab) in zip(temb, sets):
        q8.deqW16(t16, vocab, VOCAB, DIM)
    step_bytes = (DEC_LAYERS * sum(n * k + n * (k // 32) * 2 for _, n, k in DEC_SHAPES)
                  + VOCAB * DIM + VOCAB * (DIM // 32) * 2)
    res = {"workload": "batched decode step: 4 layers x (self qkv 1280->3840, self out, cross q, "
                       "cross out 1280->1280, ffn 1280->5120->1280) through the skinny Q8 "
                       "projection (f32 rows) + vocab 1280->51866 as the engine calls it "
                       "(matmulF16Batched on deqW16's recorded tok_emb copy, f16 rows in and "
                       "out), weights cold (two alternating sets)",
           "weight_bytes_per_step": step_bytes}
    from madi_amd.issue import IssueList
    for m in (8, 16):
        def step(i, m=m, lst=None):
            layers, vocab = sets[i % 2]
            q = lst if lst is not None else q8
            for ws in layers:
                for j, (_, n, k) in enumerate(DEC_SHAPES):
                    q.pproj(xin, ws[j], out, m, n, k)
            q.matmulF16Batched(x16, temb[i % 2], l16, m, VOCAB, DIM)
        step(0)
        step(1)
        tp = _timed(torch, stream, step, reps, settle=True)
        two = IssueList()   # two steps, one per weight set
        step(0, lst=two)
        step(1, lst=two)
        t = _timed_list(torch, stream, two, reps // 2, per=2)
        byts = step_bytes + DEC_LAYERS * sum(m * k * 4 + m * n * 4 for _, n, k in DEC_SHAPES) \
            + m * DIM * 2 + m * VOCAB * 2
        one = IssueList()   # one weight set every step (the engine's loop; warm)
        step(0, lst=one)
        tw = _timed_list(torch, stream, one, reps)
        res[f"m{m}"] = {"us_per_step": round(t * 1e6, 2), "gbs": round(byts / t / 1e9, 1),
                        "frac_hbm_peak": round(byts / t / 1e9 / PEAK_HBM_GBS, 4),
                        "issued_from": "C (madi_amd.issue)",
                        "python_issued_us_per_step": round(tp * 1e6, 2),
                        "warm_us_per_step": round(tw * 1e6, 2)}
        tv = _timed(torch, stream,
                    lambda i, m=m: q8.matmulF16Batched(x16, temb[i % 2], l16, m, VOCAB, DIM), reps)
        vb = VOCAB * DIM + VOCAB * (DIM // 32) * 2 + m * DIM * 2 + m * VOCAB * 2
        res[f"m{m}"]["vocab_us"] = round(tv * 1e6, 2)
        res[f"m{m}"]["vocab_frac_hbm_peak"] = round(vb / tv / 1e9 / PEAK_HBM_GBS, 4)
    # the copies were only recorded: drop the records before torch reuses
    # their memory (madi_q8_forget writes nothing)
    for t16 in temb:
        q8.forget(t16)
    del sets, temb
    m = 1500
    ctx = torch.from_numpy(synth.activations(np.random.default_rng(103), m, DIM).view(np.int16)).cuda()
    kv = torch.empty((m, 2560), dtype=torch.int16, device="cuda")
    wkv = [_upload_layer(q8, 2990 + l, 2560, DIM) for l in range(DEC_LAYERS)]
    q8.kGemmQ8(ctx, wkv[0], kv, m, 2560, DIM)
    t = _timed(torch, stream, lambda i: q8.kGemmQ8(ctx, wkv[i % DEC_LAYERS], kv, m, 2560, DIM), 20)
    fl = 2.0 * m * 2560 * DIM
    res["cross_kv_m1500"] = {"us": round(t * 1e6, 2), "tflops": round(fl / t / 1e12, 1),
                             "frac_fp16_peak": round(fl / t / 1e12 / PEAK_FP16_TFLOPS, 4)}
    return res


def config_decode_token(torch, stream, q8, reps=20):
    """One decoder token at M = 1 through the GEMV family with the reference
    decodeBlock's Q8 calls (decoder.zig:260-309): per layer the fused q|k|v
    GEMV 1280->3840 with the K/V cache store, out 1280->1280, cross-q + bias,
    cross-out, FFN-up + bias + GELU 1280->5120, FFN-down + bias + residual
    5120->1280; then the vocab logits 1280->51866 (transcribe.zig:4369).  Two
    alternating weight sets (2 x 168 MB > the 256 MB Infinity Cache).  Also
    the q|k|v GEMV alone over 64 rotating copies (315 MB), cold."""
    d, mlp = DIM, 5120
    rng = np.random.default_rng(105)
    f32 = lambda *shape: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda()
    x, xb, q, ao, mo, mh = f32(mlp), f32(d), f32(d), f32(d), f32(d), f32(mlp)
    qb, vb, bd, bm = f32(d), f32(d), f32(d), f32(mlp)
    kc, vc = f32(448, d), f32(448, d)
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    logits = torch.empty(VOCAB, dtype=torch.float32, device="cuda")
    shapes = [(3 * d, d), (d, d), (d, d), (d, d), (mlp, d), (d, mlp)]
    sets = []
    for s_ in range(2):
        layers = [[_upload_layer(q8, 4000 + 100 * s_ + 8 * l + j, n, k)
                   for j, (n, k) in enumerate(shapes)] for l in range(DEC_LAYERS)]
        sets.append((layers, _upload_layer(q8, 4900 + s_, VOCAB, DIM)))
    step_bytes = (DEC_LAYERS * sum(n * k + n * (k // 32) * 2 for n, k in shapes)
                  + VOCAB * DIM + VOCAB * (DIM // 32) * 2)

    f_gelu = q8.getFunction("gemv_q8_bias_gelu")  # the handles decoder.zig resolves once
    f_res = q8.getFunction("gemv_q8_bias_res")

    def token(i, lst=None):
        layers, vocab = sets[i % 2]
        q_ = lst if lst is not None else q8
        for w in layers:
            q_.kQkv(q, xb, w[0], qb, vb, kc, vc, pos, d)
            q_.kGemvQ8(mo, ao, w[1], d, d)
            q_.kGemvQ8Bias(q, xb, w[2], bd, d, d)
            q_.kGemvQ8(mo, ao, w[3], d, d)
            q_.kGemvQ8BiasEpi(f_gelu, mh, xb, w[4], bm, mlp, d)
            q_.kGemvQ8BiasEpi(f_res, x, mh, w[5], bd, d, mlp)
        q_.kLogitGemv(logits, vocab.qs, vocab.scales, xb, VOCAB, DIM)

    from madi_amd.issue import IssueList
    token(0)
    token(1)
    tp = _timed(torch, stream, token, reps, settle=True)
    two = IssueList()   # two tokens, one per weight set
    token(0, two)
    token(1, two)
    t = _timed_list(torch, stream, two, reps // 2, per=2)
    res = {"workload": "decoder token at M = 1: 4 layers x (q|k|v + K/V store 1280->3840, out, "
                       "cross-q + bias, cross-out 1280->1280, FFN-up + bias + GELU 1280->5120, "
                       "FFN-down + bias + residual 5120->1280) + vocab logits 1280->51866, GEMV "
                       "family, f32 activations, weights cold (two alternating sets)",
           "weight_bytes_per_token": step_bytes,
           "us_per_token": round(t * 1e6, 2), "gbs": round(step_bytes / t / 1e9, 1),
           "frac_hbm_peak": round(step_bytes / t / 1e9 / PEAK_HBM_GBS, 4),
           "issued_from": "C (madi_amd.issue)",
           "python_issued_us_per_token": round(tp * 1e6, 2)}
    # the engine's decode loop re-reads ONE weight set every token (the 168 MB
    # fit the 256 MB Infinity Cache): the same calls on set 0 only
    one = IssueList()
    token(0, one)
    tw = _timed_list(torch, stream, one, reps)
    res["warm"] = {"what": "one weight set re-read every token, as the engine's decode loop does "
                           "(168 MB, resident in the Infinity Cache)",
                   "us_per_token": round(tw * 1e6, 2),
                   "gbs": round(step_bytes / tw / 1e9, 1)}
    del sets
    base = _upload_layer(q8, 4990, 3 * d, d)
    ws = []
    for _ in range(64):  # distinct device copies of one weight
        tq, ts = (t_.clone() for t_ in base._keep)
        ws.append(q8.Q8(tq.data_ptr(), ts.data_ptr(), (tq, ts)))
    q8.kQkv(q, xb, ws[0], qb, vb, kc, vc, pos, d)
    rot = IssueList()   # the 64 copies in turn, issued from C (a ~4 us kernel)
    for w in ws:
        rot.kQkv(q, xb, w, qb, vb, kc, vc, pos, d)
    tq = _timed_list(torch, stream, rot, 2, per=64)
    qb_bytes = 3 * d * d + 3 * d * (d // 32) * 2
    res["qkv_gemv"] = {"us": round(tq * 1e6, 2), "gbs": round(qb_bytes / tq / 1e9, 1),
                       "frac_hbm_peak": round(qb_bytes / tq / 1e9 / PEAK_HBM_GBS, 4)}
    return res


def config_prefill(torch, stream, q8, reps=24):
    """Sequence prefill at its largest M = 320 rows (prefillBlock,
    decoder.zig:473-495): one decoder layer's pproj calls, q|k|v 1280->3840,
    out, cross-q, cross-out 1280->1280, FFN 1280->5120->1280, f32 rows in and
    out; weights cold (24 rotating copies of each)."""
    from madi_amd import synth
    m = 320
    res = {"workload": "sequence prefill M=320: one decoder layer's batched projections "
                       "(pproj: q|k|v 1280->3840, out, cross-q, cross-out 1280->1280, FFN "
                       "1280->5120->1280), f32 in/out, cold weights"}
    total = 0.0
    flops = 0.0
    for name, n, k in (("qkv", 3840, 1280), ("out", 1280, 1280), ("cross_q", 1280, 1280),
                       ("cross_out", 1280, 1280), ("ffn_up", 5120, 1280), ("ffn_down", 1280, 5120)):
        base = _upload_layer(q8, 5000 + n + k, n, k)
        ws = []
        for _ in range(24):
            tq, ts = (t_.clone() for t_ in base._keep)
            ws.append(q8.Q8(tq.data_ptr(), ts.data_ptr(), (tq, ts)))
        x = torch.from_numpy(np.random.default_rng(n).standard_normal((m, k)).astype(np.float32)).cuda()
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        q8.pproj(x, ws[0], out, m, n, k)
        t = _timed(torch, stream, lambda i: q8.pproj(x, ws[i % 24], out, m, n, k), reps)
        fl = 2.0 * m * n * k
        res[name] = {"us": round(t * 1e6, 2), "tflops": round(fl / t / 1e12, 1)}
        total += t
        flops += fl
    res["us_per_layer"] = round(total * 1e6, 2)
    res["tflops"] = round(flops / total / 1e12, 1)
    res["frac_fp16_peak"] = round(flops / total / 1e12 / PEAK_FP16_TFLOPS, 4)
    return res


def config_long_audio(torch, stream, q8, reps=5):
    """16 stacked 30 s windows: fc1 M=24000 K=1280 N=5120 and fc2 M=24000
    K=5120 N=1280 Q8 GEMMs."""
    import torch as _t  # noqa: F401
    m = 24000
    g = torch.Generator(device="cuda").manual_seed(104)
    a = torch.randn((m, 5120), generator=g, device="cuda", dtype=torch.float32).half().view(torch.int16)
    c = torch.empty((m, 5120), dtype=torch.int16, device="cuda")
    res = {"workload": "fc1 M=24000 K=1280 N=5120, fc2 M=24000 K=5120 N=1280 Q8 GEMMs "
                       "(activations drawn on the device: torch Philox N(0,1) -> f16)"}
    res["clocks"] = ("first: one launch after 0.2 s idle (the clock the chip starts a "
                     "window at); sustained: the average of 5 launches after 8 untimed ones "
                     "back to back (the clock it settles to under continuous MFMA load)")
    for name, n, k in (("fc1", 5120, 1280), ("fc2", 1280, 5120)):
        w = _upload_layer(q8, 3000 + n, n, k)
        q8.kGemmQ8(a, w, c, m, n, k)
        torch.cuda.synchronize()
        time.sleep(0.2)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        q8.kGemmQ8(a, w, c, m, n, k)
        e1.record(stream)
        torch.cuda.synchronize()
        t1 = e0.elapsed_time(e1) * 1e-3
        for _ in range(8):
            q8.kGemmQ8(a, w, c, m, n, k)
        t = _timed(torch, stream, lambda i: q8.kGemmQ8(a, w, c, m, n, k), reps)
        fl = 2.0 * m * n * k
        res[name] = {"us": round(t * 1e6, 1), "tflops": round(fl / t / 1e12, 1),
                     "frac_fp16_peak": round(fl / t / 1e12 / PEAK_FP16_TFLOPS, 4),
                     "first_launch_us": round(t1 * 1e6, 1),
                     "first_launch_frac_fp16_peak": round(fl / t1 / 1e12 / PEAK_FP16_TFLOPS, 4)}
    return res


def measured_traffic():
    """HBM bytes per launch {kernel: bytes} from the committed PMC summary, if any."""
    out = {}
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch"):
                for kv in line.split()[1:]:
                    k, v = kv.split("=")
                    out[k] = float(v)
    except OSError:
        pass
    return out


def calibrate_copy():
    import torch
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": 5}))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def config_encoder_attention(torch, stream, q8, reps=50):
    """The encoder self-attention of one 30 s window over its Q, K, V
    projections (the kFlash call, engine/metal/encoder.zig:138-152): 1500
    frames x 20 heads x head dim 64, f16, one layer.  FLOPs = 4 seq^2 64 heads
    (Q K^T and P V; the softmax is not counted), against the fp16 MFMA peak."""
    seq, nh = q8.ENC_SEQ, q8.NH
    g = torch.Generator(device="cuda").manual_seed(200)
    q, k, v = (torch.randn(seq, nh * 64, device="cuda", generator=g).half() for _ in range(3))
    o = torch.empty_like(q)
    f = q8.getFunction("m4_flash_enc")

    def one(_):
        q8.kFlash(f, o, q, k, v, seq, nh)

    one(0)
    t = _timed(torch, stream, one, reps)
    flops = 4.0 * seq * seq * 64 * nh
    return {
        "workload": "encoder self-attention, 1500 frames x 20 heads x 64, f16 Q/K/V/out, one layer",
        "us": round(t * 1e6, 2), "gflop": round(flops / 1e9, 3),
        "tflops": round(flops / t / 1e12, 1),
        "frac_fp16_peak": round(flops / t / 1e12 / PEAK_FP16_TFLOPS, 4),
    }


CONFIGS = {
    "encoder_window": config_encoder_window,
    "encoder_window_engine": config_encoder_window_engine,
    "encoder_window_f16cache": config_encoder_window_f16cache, "batched_decode": config_batched_decode,
    "decode_token": config_decode_token, "prefill": config_prefill,
    "long_audio": config_long_audio, "encoder_attention": config_encoder_attention,
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the encoder-window, batched-decode, decoder-token and long-audio "
                         "measurements")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (PMC calibration)")
    ap.add_argument("--config", choices=sorted(CONFIGS),
                    help="only run this one configuration and print its JSON (for profiling "
                         "one workload's kernels)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): the Q8 matmul "
              "path is built and measured on a single MI355X (one GPU's share of the work); "
              "sharding it over several GPUs is a design, not a built path.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import madi_amd.q8 as q8
    from madi_amd import synth

    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    q8.init(stream)
    dev_name = torch.cuda.get_device_name(0)
    if args.config:
        log(f"device {dev_name}; configuration {args.config} only")
        print(json.dumps({"config": args.config, "device": dev_name,
                          **CONFIGS[args.config](torch, stream, q8)}))
        return
    log(f"device {dev_name}; preparing inputs")

    a, qs, sc = synth.gemm_case(0, M, N, K)
    wg = q8.upload_q8(qs, sc)
    da = torch.from_numpy(a.view(np.int16)).cuda()
    dc = torch.empty((M, N), dtype=torch.int16, device="cuda")

    x16, qv, sv = synth.gemv_case(1, VOCAB, DIM)
    dx = torch.from_numpy(x16.view(np.int16)).cuda()
    wv = [q8.upload_q8(qv, sv) for _ in range(GEMV_COPIES)]  # distinct HBM copies
    dlog = torch.empty(VOCAB, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    def gemm(i):
        q8.kGemmQ8(da, wg, dc, M, N, K)

    def gemv(i):
        q8.gemv_f16x(dlog, dx, wv[i % GEMV_COPIES], VOCAB, DIM)

    dx32 = torch.from_numpy(x16.astype(np.float32)).cuda()

    def logit(i):  # the engine's kLogitGemv: f32 activations (transcribe.zig:4369)
        q8.kLogitGemv(dlog, wv[i % GEMV_COPIES].qs, wv[i % GEMV_COPIES].scales, dx32, VOCAB, DIM)

    log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        gemm(i)
        gemv(i)
        logit(i)
    torch.cuda.synchronize()

    # One step: the fc1 GEMM, the engine's f32-activation vocab GEMV and the
    # vocab GEMV with fp16 activations.  The three loops run back to back in
    # one synchronised region, each timed by events on the stream.  (Of two
    # GEMV loops after the GEMMs the second runs ~0.2 us per launch slower,
    # whichever kernel it holds; the engine's call takes the first place.)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(args.steps):
        gemm(i)
    ev[1].record(stream)
    for i in range(args.steps):
        logit(i)
    ev[2].record(stream)
    for i in range(args.steps):
        gemv(i)
    ev[3].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    g_avg = ev[0].elapsed_time(ev[1]) * 1e-3 / args.steps   # s per GEMM launch
    l_avg = ev[1].elapsed_time(ev[2]) * 1e-3 / args.steps   # s per f32-x GEMV launch
    v_avg = ev[2].elapsed_time(ev[3]) * 1e-3 / args.steps   # s per GEMV launch
    l_gbs = (gemv_bytes() + DIM * 2) / l_avg / 1e9              # x is f32: 2 more bytes per element
    gemm_tflops = gemm_flops() / g_avg / 1e12
    gemv_gbs = gemv_bytes() / v_avg / 1e9
    ms_per_step = wall / args.steps * 1e3
    traffic = measured_traffic()
    log(f"gemm {g_avg*1e6:.2f} us ({gemm_tflops:.1f} TFLOP/s), gemv {v_avg*1e6:.2f} us "
        f"({gemv_gbs:.0f} GB/s), f32-x gemv {l_avg*1e6:.2f} us ({l_gbs:.0f} GB/s), "
        f"wall {ms_per_step:.3f} ms/step")

    result = {
        "metric": "Q8 GEMM TFLOP/s @1500x1280x5120 + Q8 GEMV GB/s @vocab; % of roofline",
        "value": round(gemm_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16xi8->f32acc",
        "data": "synthetic (numpy PCG64 seed 0/1: A~N(0,1) f16, q~U{-127..127}, s~f16(U[1e-3,1e-2]))",
        "config": {
            "workload": "encoder fc1 Q8 GEMM 1500x1280->5120 (f16 out; one weight copy, warm: "
                        "resident in the Infinity Cache across launches; cold per-layer figures "
                        "under configs.encoder_window) + decoder vocab Q8 GEMV 1x1280->51866 "
                        "(f32 out, 4 rotating cold weight copies)",
            "gemm_mnk": [M, N, K], "gemv_nk": [VOCAB, DIM], "device": dev_name,
        },
        "roofline": {
            "bound": "mfma", "achieved": round(gemm_tflops, 2), "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic.get("q8_gemm_kernel"), "kernel": "q8_gemm_kernel",
            "avg_us": round(g_avg * 1e6, 3),
            "algorithmic_per_launch": gemm_flops(),
        },
        "gemv": {
            "value": round(gemv_gbs, 1), "unit": "GB/s",
            "roofline": {
                "bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(gemv_gbs / PEAK_HBM_GBS, 4),
                "traffic": traffic.get("q8_gemv_kernel"), "kernel": "q8_gemv_kernel",
                "avg_us": round(v_avg * 1e6, 3),
                "algorithmic_per_launch": gemv_bytes(),
            },
            "engine_f32x": {
                "what": "kLogitGemv as the engine calls it (f32 activations, "
                        "madi_q8_logit_gemv), same cold rotation",
                "avg_us": round(l_avg * 1e6, 3), "gbs": round(l_gbs, 1),
                "frac": round(l_gbs / PEAK_HBM_GBS, 4),
            },
        },
    }
    if not args.no_configs:
        log("encoder window (32 layers x 4 GEMMs at M=1500)")
        cfg = {"encoder_window": config_encoder_window(torch, stream, q8)}
        log("encoder window as the engine issues it (32 layers x 6 GEMMs at M=1500)")
        cfg["encoder_window_engine"] = config_encoder_window_engine(torch, stream, q8)
        log("encoder window in the F16-cache mode (32 layers x 6 GEMMs on F16 weights)")
        cfg["encoder_window_f16cache"] = config_encoder_window_f16cache(torch, stream, q8)
        log("batched decode (M=8, 16)")
        cfg["batched_decode"] = config_batched_decode(torch, stream, q8)
        log("decoder token (M=1, GEMV family)")
        cfg["decode_token"] = config_decode_token(torch, stream, q8)
        log("sequence prefill (M=320)")
        cfg["prefill"] = config_prefill(torch, stream, q8)
        log("long audio (M=24000)")
        cfg["long_audio"] = config_long_audio(torch, stream, q8)
        log("encoder self-attention (1500 x 20 heads)")
        cfg["encoder_attention"] = config_encoder_attention(torch, stream, q8)
        result["configs"] = cfg
    if not args.no_cpu:
        threads = cpu_share()
        log(f"cpu baseline on {threads} threads ({cpu_model()}, nproc {os.cpu_count()})")
        cb = cpu_baseline(threads)
        result["cpu_baseline"] = {
            "value": round(cb["gemm_nt_tflops"], 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "sample": cb["sample"], "cpu": cpu_model(),
            "nproc": os.cpu_count(), "runs": 5, "median": True, "build": cb["build"],
            "label": "reference CPU path (restated), baseline only",
            "single_thread": {"value": round(cb["gemm_1t_tflops"], 6), "unit": "TFLOP/s",
                              "cores": 1},
            "gemv": {"value": round(cb["gemv_nt_gbs"], 2), "unit": "GB/s", "cores": threads,
                     "single_thread_gbs": round(cb["gemv_1t_gbs"], 2)},
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
