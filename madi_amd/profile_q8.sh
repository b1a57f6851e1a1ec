#!/bin/bash
# rocprofv3 runs behind profiles/: the kernel trace of bench.py's headline
# (fc1 Q8 GEMM + vocab Q8 GEMV), HBM traffic (FETCH_SIZE and WRITE_SIZE in
# separate passes, each calibrated on a 256 MiB device copy) and MFMA
# utilisation counters of the same launches, plus the kernel trace of every
# configuration.  Raw output goes under $1 (default gpurun_out/prof).
set -o pipefail
R=$(cd "$(dirname "$0")/.." && pwd)
mkdir -p "${1:-$R/gpurun_out/prof}"
O=$(cd "${1:-$R/gpurun_out/prof}" && pwd)
cd /tmp && export TMPDIR=/tmp
B="python3 $R/bench.py --steps 50 --warmup 10 --no-cpu --no-configs"
step() { echo "[profile] $1" >&2; }
step "kernel trace (headline)"
timeout -s KILL 240 rocprofv3 --kernel-trace --stats --output-format csv -d "$O/kt" -o run -- $B > "$O/kt.log" 2>&1 || exit 1
step "kernel trace (all configurations)"
timeout -s KILL 300 rocprofv3 --kernel-trace --stats --output-format csv -d "$O/kt_all" -o run -- python3 $R/bench.py --no-cpu > "$O/kt_all.log" 2>&1 || exit 2
P="python3 $R/bench.py --steps 10 --warmup 2 --no-cpu --no-configs"
C="python3 $R/bench.py --calibrate-copy"
for ctr in FETCH_SIZE WRITE_SIZE; do
  step "pmc $ctr"
  timeout -s KILL 90 rocprofv3 --pmc $ctr --output-format csv -d "$O/pmc_$ctr" -o run -- $P > "$O/pmc_$ctr.log" 2>&1 || exit 3
  timeout -s KILL 90 rocprofv3 --pmc $ctr --output-format csv -d "$O/cal_$ctr" -o run -- $C > "$O/cal_$ctr.log" 2>&1 || exit 4
done
step "pmc MFMA utilisation"
timeout -s KILL 90 rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 GRBM_GUI_ACTIVE --output-format csv -d "$O/pmc_mfma" -o run -- $P > "$O/pmc_mfma.log" 2>&1 || exit 5
step "done"
