"""Build recipe for the gfx950 Q8 matmul library (libmadi_q8.so).

Compiles every HIP source under madi_amd/csrc with hipcc for gfx950 only and
links them into one shared library next to this file, so the built library
travels with the source tree.  Run as `python -m madi_amd.build`.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmadi_q8.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU forms are kept out of every kernel: the library does its
# fp32 work in scalar or vector-of-scalar code and lets no v_pk_*_f32 appear.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading kernel arguments arrive in SGPRs at wave launch (gfx950 kernarg
    # preload) instead of through a scalar load after the start of the kernel
    # (0.2 - 0.8 us on the path to a kernel's first memory access).  The kernels take
    # scalar arguments in the order of first use for this.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


ISSUE_SRC = os.path.join(CSRC, "issue.c")
ISSUE_LIB = os.path.join(HERE, "libmadi_issue.so")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build_issue(lib: str = LIB, out: str = ISSUE_LIB) -> str:
    """The compiled issue loop (csrc/issue.c) that bench.py uses to replay a
    call list from C, linked against the library it calls."""
    tmp = out + ".tmp"
    _run(["gcc", "-O2", "-std=c11", "-shared", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include"),
          ISSUE_SRC, "-o", tmp, "-L", os.path.dirname(lib), "-l:" + os.path.basename(lib),
          "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}")
    return err


def build(verbose: bool = False, extra_flags=(), out: str = LIB, obj_dir: str = OBJ_DIR) -> str:
    """Compile all sources and link the library (default libmadi_q8.so next to
    this file); `extra_flags` (e.g. -D tuning macros) go to every compile."""
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o") for src in srcs]
    # one hipcc per source, at most 8 at a time
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        msgs = list(pool.map(lambda so: _run([HIPCC, *HIP_FLAGS, *extra_flags, "-c", so[0], "-o", so[1]]),
                             zip(srcs, objs)))
    if verbose:
        for msg in msgs:
            if msg.strip():
                print(msg)
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(tmp, out)
    if out == LIB:
        build_issue()
    return out


if __name__ == "__main__":
    print(build(verbose=True))
