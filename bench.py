"""Benchmark of the MI355X Q8 matmul path (one GPU).

A step is one pass of the hot path over one batch of synthetic input:
  1. the encoder fc1 Q8 GEMM, A f16 [1500, 1280] x W int8 [5120, 1280] (+ fp16
     per-32 scales) -> C f16 [1500, 5120], fp32 accumulation, and
  2. the decoder vocab-logit Q8 GEMV, x f16 [1280] x W int8 [51866, 1280] ->
     f32 logits [51866], cold: the step cycles through 4 distinct weight copies
     (4 x 70.75 MB > the 256 MB Infinity Cache) so each launch streams HBM.
Inputs are resident in HBM before the timed region.  The timed region runs
the K steps' GEMMs back to back and then their GEMVs, with HIP events on the
kernels' stream at the start, between the two runs and at the end, so each
kernel's average duration is (event span) / K -- the figure rocprofv3's
kernel trace reports for the same launches (a per-launch event pair would add
the dispatch gap).  The JSON line reports the GEMM as the headline value
(TFLOP/s) and the GEMV beside it (GB/s), each with its roofline fraction and,
when profiles/traffic_q8_fc1_gemm_vocab_gemv.md holds them, the measured HBM
bytes per launch, plus the restated reference CPU path timed on this host's
cores (a reported baseline only).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
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


def cpu_baseline(threads: int):
    """The oracle (C restatement of the reference's CPU loop,
    engine/metal/test_q8gemm.zig:59-69) on a bounded row sample of the same
    fc1 workload, and the vocab GEMV in full; single thread and `threads`."""
    import oracle as O
    from madi_amd import synth
    a, qs, sc = synth.gemm_case(0, M, N, K)
    res = {}
    rows1 = np.arange(0, M, 3, dtype=np.uint32)[:480]
    O.q8_gemm_rows(a, qs, sc, rows=rows1[:2], threads=1)  # warm-up
    t = time.perf_counter()
    O.q8_gemm_rows(a, qs, sc, rows=rows1, threads=1)
    dt1 = time.perf_counter() - t
    rowsn = np.arange(0, M, dtype=np.uint32)
    t = time.perf_counter()
    O.q8_gemm_rows(a, qs, sc, rows=rowsn, threads=threads)
    dtn = time.perf_counter() - t
    f_row = 2.0 * N * K
    res["gemm_1t_tflops"] = f_row * rows1.size / dt1 / 1e12
    res["gemm_nt_tflops"] = f_row * rowsn.size / dtn / 1e12
    x, qv, sv = synth.gemv_case(0, VOCAB, DIM)
    xf = x.astype(np.float32)
    t = time.perf_counter()
    for _ in range(3):
        O.q8_gemv(xf, qv, sv, threads=1)
    dtv1 = (time.perf_counter() - t) / 3
    t = time.perf_counter()
    for _ in range(10):
        O.q8_gemv(xf, qv, sv, threads=threads)
    dtvn = (time.perf_counter() - t) / 10
    res["gemv_1t_gbs"] = gemv_bytes() / dtv1 / 1e9
    res["gemv_nt_gbs"] = gemv_bytes() / dtvn / 1e9
    res["sample"] = (f"fc1 GEMM: {rows1.size} of {M} rows single-thread ({dt1:.1f} s, rate per row) "
                     f"and all {rowsn.size} rows on {threads} threads ({dtn:.1f} s); vocab GEMV: "
                     f"full 1x{DIM}x{VOCAB}, 3 runs single-thread, 10 on {threads} threads")
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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (PMC calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): the Q8 matmul "
              "path runs on a single MI355X; see DESIGN.md for how it would shard.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import madi_amd.q8 as q8
    from madi_amd import synth

    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    q8.init(stream)
    dev_name = torch.cuda.get_device_name(0)
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

    log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        gemm(i)
        gemv(i)
    torch.cuda.synchronize()

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(args.steps):
        gemm(i)
    ev[1].record(stream)
    for i in range(args.steps):
        gemv(i)
    ev[2].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    g_avg = ev[0].elapsed_time(ev[1]) * 1e-3 / args.steps   # s per GEMM launch
    v_avg = ev[1].elapsed_time(ev[2]) * 1e-3 / args.steps   # s per GEMV launch
    gemm_tflops = gemm_flops() / g_avg / 1e12
    gemv_gbs = gemv_bytes() / v_avg / 1e9
    ms_per_step = wall / args.steps * 1e3
    traffic = measured_traffic()
    log(f"gemm {g_avg*1e6:.2f} us ({gemm_tflops:.1f} TFLOP/s), gemv {v_avg*1e6:.2f} us "
        f"({gemv_gbs:.0f} GB/s), wall {ms_per_step:.3f} ms/step")

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
            "workload": "encoder fc1 Q8 GEMM 1500x1280->5120 (f16 out) + decoder vocab Q8 GEMV "
                        "1x1280->51866 (f32 out, 4 rotating cold weight copies)",
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
        },
    }
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        log(f"cpu baseline on {threads} threads ({cpu_model()})")
        cb = cpu_baseline(threads)
        result["cpu_baseline"] = {
            "value": round(cb["gemm_nt_tflops"], 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "sample": cb["sample"], "cpu": cpu_model(),
            "single_thread": {"value": round(cb["gemm_1t_tflops"], 6), "unit": "TFLOP/s",
                              "cores": 1},
            "gemv": {"value": round(cb["gemv_nt_gbs"], 2), "unit": "GB/s", "cores": threads,
                     "single_thread_gbs": round(cb["gemv_1t_gbs"], 2)},
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
