"""Every instance of the hand-scheduled Q8 GEMM kernel (madi_amd/csrc/gemm.hip)
is free of vmcnt races on its K-loop path: no instruction touches a VGPR that
an outstanding vector-memory load is still filling.  Compiles the kernel to
gfx950 assembly (CPU only) and simulates the in-order vmcnt queue."""
import os
import shutil
import subprocess

import pytest

from isa_vmcnt import hazards, kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    from madi_amd.build import HIP_FLAGS
    out = tmp_path_factory.mktemp("isa") / "gemm.s"
    src = os.path.join(ROOT, "madi_amd", "csrc", "gemm.hip")
    flags = [f for f in HIP_FLAGS if f != "-fPIC"]
    subprocess.run([HIPCC, *flags, "--cuda-device-only", "-S", src, "-o", str(out)],
                   check=True, capture_output=True)
    return kernels(out.read_text())


def test_every_gemm_instance_is_race_free(gemm_asm):
    names = [n for n in gemm_asm if "q8_gemm_kernel" in n]
    # MT 1-4 x 3 epilogues x padded or not, the m-tile-major tail instances
    # (MT 2-4 x 3 epilogues), the 128-column instances (MT 2 and 4 x 3
    # epilogues), and the f32-in/f32-out instances of the batched projection
    # (MT 1-2, no epilogue, padded or not, and MT 1-2 on 128-column tiles)
    assert len(names) == 45, names
    bad = {n: hazards(gemm_asm[n])[:3] for n in names}
    bad = {n: b for n, b in bad.items() if b}
    assert not bad, bad


def test_every_ksplit_instance_is_race_free(gemm_asm):
    """The in-workgroup K split (q8_gemm_ks_kernel, one instance per
    epilogue): prologue, peeled first trip, K loop, last trip, reduction."""
    names = [n for n in gemm_asm if "q8_gemm_ks_kernel" in n]
    assert len(names) == 3, names
    bad = {n: hazards(gemm_asm[n])[:3] for n in names}
    bad = {n: b for n, b in bad.items() if b}
    assert not bad, bad


def test_every_persistent_instance_is_race_free(gemm_asm):
    """The persistent tile loop (q8_gemm_persist_kernel, one instance per
    epilogue): two trips of the tile loop, each with the K loop three times,
    the next tile's prologue issued before the finished tile's epilogue."""
    names = [n for n in gemm_asm if "q8_gemm_persist_kernel" in n]
    assert len(names) == 3, names
    bad = {n: hazards(gemm_asm[n])[:3] for n in names}
    bad = {n: b for n, b in bad.items() if b}
    assert not bad, bad


@pytest.fixture(scope="module")
def attn_asm(tmp_path_factory):
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    from madi_amd.build import HIP_FLAGS
    out = tmp_path_factory.mktemp("isa") / "attn.s"
    src = os.path.join(ROOT, "madi_amd", "csrc", "attn.hip")
    flags = [f for f in HIP_FLAGS if f != "-fPIC"]
    subprocess.run([HIPCC, *flags, "--cuda-device-only", "-S", src, "-o", str(out)],
                   check=True, capture_output=True)
    return kernels(out.read_text())


def test_every_attention_instance_is_race_free(attn_asm):
    """The encoder attention kernel (one to four key groups, pipelined and
    plain schedules): the Q fragments loaded into registers are not touched
    before their wait, on any of the prologue's paths, and the block loop adds
    no register loads."""
    names = [n for n in attn_asm if "flash_enc_kernel" in n]
    assert len(names) == 4, names
    bad = {n: hazards(attn_asm[n])[:3] for n in names}
    bad = {n: b for n, b in bad.items() if b}
    assert not bad, bad


def test_wait_check_catches_a_premature_read():
    """The wait check itself: a read of a load's destination before its wait,
    and a register reused while a dead load is in flight, are both flagged;
    the waited read is not."""
    asm = ["buffer_load_dwordx4 v[4:7], v1, s[0:3], s4 offen",
           "buffer_load_dwordx4 v[8:11], v1, s[0:3], s5 offen",
           "s_waitcnt vmcnt(1)",
           "v_add_u32 v12, v4, v5",      # fine: v[4:7] has landed
           "v_add_u32 v13, v8, v9",      # premature: v[8:11] is still in flight
           "v_mov_b32 v10, 0",           # reuse of an in-flight register
           "s_waitcnt vmcnt(0)",
           "v_add_u32 v14, v8, v9",
           "s_endpgm"]
    bad = hazards(asm)
    assert [b[2] for b in bad] == ["v_add_u32 v13, v8, v9", "v_mov_b32 v10, 0"], bad
