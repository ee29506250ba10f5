"""libdmc_hip on the CPU: the C ABI loads and exports every declared symbol,
and the host-side logic that needs no device behaves as specified.  No GEMV is
computed here (there is no GPU); device-free entry points only.
"""
import os
import pathlib
import re
import subprocess
import sys

import numpy as np
import pytest

import demonic_amd as d
from demonic_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "dmc_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dmc_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.SIGNATURES), \
        set(declared_functions()) ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (dmc_\w+)", out))
    assert set(declared_functions()) <= exported


def test_reference_operator_surface_is_exported_with_reference_names():
    # compiler/src/gpu.rs:400, 421, 449, 468
    for name in ("dmc_matmul_bf16_gpu", "dmc_matmul_bf16_gpu_batched",
                 "dmc_matmul_bf16_gpu_batched_deferred", "dmc_matmul_bf16_gpu_flush"):
        assert name in declared_functions()
    assert _lib.SIGNATURES["dmc_matmul_bf16_gpu"][1] == [_lib.i64] * 6
    assert _lib.SIGNATURES["dmc_matmul_bf16_gpu_batched"][1] == [_lib.i64] * 9


def test_library_is_gfx950_code_only(tmp_path):
    """The code object bundled in our own build targets gfx950 and nothing else."""
    fb = tmp_path / "fatbin.bin"
    r = subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin",
                        str(_lib.LIB_PATH), str(fb)], capture_output=True, text=True)
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                          f"--input={fb}"], capture_output=True, text=True)
    if r.returncode != 0 or out.returncode != 0:
        pytest.skip("offload bundle tools unavailable")
    targets = [t for t in out.stdout.split() if "amdgcn" in t]
    assert targets == ["hipv4-amdgcn-amd-amdhsa--gfx950"], out.stdout


def _kernel_descriptors(tmp_path):
    """The AMDGPU metadata of every kernel in our own build's gfx950 code
    object (llvm-readelf --notes), or None when the tools are missing."""
    import yaml
    fb, co = tmp_path / "fatbin.bin", tmp_path / "k.co"
    steps = (["objcopy", "-O", "binary", "--only-section=.hip_fatbin", str(_lib.LIB_PATH), str(fb)],
             ["/opt/rocm/llvm/bin/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fb}",
              "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"])
    for cmd in steps:
        if subprocess.run(cmd, capture_output=True).returncode != 0:
            return None
    r = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "--notes", str(co)], capture_output=True, text=True)
    if r.returncode != 0 or "amdhsa.kernels" not in r.stdout:
        return None
    t = r.stdout
    a = t.index("\n", t.index("---")) + 1
    return yaml.safe_load(t[a:t.index("\n...", a)])["amdhsa.kernels"]


def test_kernel_descriptors_within_dispatch_limits(tmp_path):
    """Every kernel's dispatch needs stay inside what an AQL dispatch packet
    and a gfx950 CU allow: static LDS <= 160 KiB, no scratch (private
    segment 0, no dynamic stack), at most 1024 work-items, kernel arguments
    well under HIP's 4 KiB.  (The check behind the finding that the queue
    aborts seen with HIP-graph replays under rocprofv3 have no cause in the
    launch parameters: every node of those graphs is one of these kernels,
    launched with a grid whose work-item count fits 32 bits,
    test_decode_step_grids_fit_a_dispatch_packet.)"""
    ks = _kernel_descriptors(tmp_path)
    if ks is None:
        pytest.skip("offload bundle tools unavailable")
    assert len(ks) > 100
    for k in ks:
        name = k[".name"]
        assert k[".group_segment_fixed_size"] <= 160 * 1024, name
        assert k[".private_segment_fixed_size"] == 0 and not k[".uses_dynamic_stack"], name
        assert k[".max_flat_workgroup_size"] <= 1024, name
        assert k[".kernarg_segment_size"] <= 1024, name
        assert k[".vgpr_spill_count"] == 0, name
        assert k[".wavefront_size"] == 64, name


def test_decode_step_grids_fit_a_dispatch_packet():
    """The launches of a C3 decode step (single and grouped, as bench.py
    captures them into HIP graphs): each plan has a nonzero grid whose
    work-item count fits the packet's 32-bit grid size, and a workgroup of
    at most 1024 work-items."""
    from demonic_amd import workloads as W
    for nm, n, k in W.LLAMA3_8B_LAYER:
        p = d.plan("rd", 1, k, n, x_addr=256, w_addr=256)
        threads = 64 * p.waves
        assert 0 < p.grid_x and 0 < threads <= 1024, (nm, p)
        assert p.grid_x * threads < 2 ** 32, (nm, p)


# ---- the route predicate (shape of jit.rs:39087-39113) ----------------------------------

def test_selection_predicate():
    sel = d.gemv_selected
    assert sel(True, 0, 1, 512, 512), "eligible GEMV refused"
    assert not sel(False, 0, 1, 512, 512), "selected with the flag off"
    assert not sel(True, 1, 1, 512, 512), "selected inside @deterministic"
    assert not sel(True, 3, 1, 4096, 14336), "nested @deterministic"
    assert not sel(True, 0, 1, 64, 128), "small GEMV selected"
    assert sel(True, 0, 1, 128, 128), "the measured crossover, k*n = 2^14"
    assert sel(True, 0, 1, 1, d.MIN_MACS), "at the threshold"
    assert not sel(True, 0, 1, 1, d.MIN_MACS - 1), "one under the threshold"
    assert sel(True, 0, 64, 64, 64), "threshold is a MAC count, not per-dimension"
    assert not sel(True, 0, 0, 4096, 4096) and not sel(True, 0, 1, 0, 4096)


# ---- launch planning (pure host computation) ----------------------------------------------

@pytest.mark.parametrize("k,align,vec", [(4096, 256, 8), (4100, 256, 4), (4098, 256, 2),
                                         (4097, 256, 1), (4096, 258, 1), (4096, 260, 2),
                                         (4096, 264, 4)])
def test_rowdot_vector_width_follows_alignment(k, align, vec):
    p = d.plan("rd", 1, k, 14336, x_addr=256, w_addr=align)
    assert p.vec == vec, p


def test_rowdot_plans_at_decode_shapes(monkeypatch):
    # streaming kernel: 8 waves split k = 4096 one 8-element vector per lane,
    # 4 weight rows per workgroup, 2 per step
    up = d.plan("rd", 1, 4096, 14336, x_addr=256, w_addr=256)
    assert (up.vec, up.waves, up.slices, up.rows_per_group, up.rows_or_rw, up.mt, up.grid_x) == \
        (8, 8, 1, 4, 2, 1, 3584)
    # long rows: workgroups of 16 rows sharing one LDS copy of x (one per CU):
    # up to K = 14336 one group of 14 waves, 2 vectors per lane ...
    down = d.plan("rd", 1, 14336, 4096, x_addr=256, w_addr=256)
    assert (down.waves, down.slices, down.rows_per_group, down.grid_x) == (14, 2, 16, 256)
    # ... beyond it (or with DMC_HIP_RD_X14=0) two 8-wave halves, ceil(K / 4096) vectors per lane ...
    assert d.plan("rd", 1, 16384, 4096, x_addr=256, w_addr=256).waves == 16
    monkeypatch.setenv("DMC_HIP_RD_X14", "0")
    down = d.plan("rd", 1, 14336, 4096, x_addr=256, w_addr=256)
    assert (down.waves, down.slices, down.rows_per_group, down.grid_x) == (16, 4, 16, 256)
    monkeypatch.delenv("DMC_HIP_RD_X14")
    # ... or, switched off, 8-wave workgroups of 8 rows, each with x in registers
    monkeypatch.setenv("DMC_HIP_RD_XLDS", "0")
    down = d.plan("rd", 1, 14336, 4096, x_addr=256, w_addr=256)
    assert (down.waves, down.slices, down.rows_per_group, down.grid_x) == (8, 4, 8, 512)
    monkeypatch.delenv("DMC_HIP_RD_XLDS")
    # fewer rows than one 16-row workgroup per CU, or a partial last round of
    # them (one 16-wave workgroup fills a CU): the 8-wave layout
    assert d.plan("rd", 1, 14336, 1024, x_addr=256, w_addr=256).waves == 8
    assert d.plan("rd", 1, 11008, 4097, x_addr=256, w_addr=256).waves == 8
    assert d.plan("rd", 1, 8192, 8192, x_addr=256, w_addr=256).waves == 14      # two whole rounds
    assert d.plan("rd", 1, 8192, 28672, x_addr=256, w_addr=256).waves == 14     # seven
    # small grids at one window per lane: 4 rows in one step, 4 per workgroup
    # (k/v projections: 256 workgroups; C1: 1024); up to 8 such workgroups
    # per CU, then 2 rows per step (C2 up/gate above)
    small = d.plan("rd", 1, 4096, 1024, x_addr=256, w_addr=256)
    assert (small.rows_or_rw, small.rows_per_group, small.grid_x) == (4, 4, 256), small
    # one GPU's gate/up share under TP = 8, 1792 = 7 * 256 rows: one 8-wave group of 7 rows per CU
    # (the streaming kernel's 4-row workgroups with DMC_HIP_RD_X8=0)
    p = d.plan("rd", 1, 4096, 1792, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.rows_per_group, p.grid_x) == (7, 7, 256), p
    for n, r in ((1024, 4), (1536, 6), (2560, 10), (3584, 14)):
        p = d.plan("rd", 1, 4096, n, x_addr=256, w_addr=256)
        assert (p.waves, p.rows_or_rw, p.rows_per_group, p.grid_x) == (8, r if r <= 8 else r // 2, r, 256), p
    assert d.plan("rd", 1, 4096, 1280, x_addr=256, w_addr=256).rows_per_group == 4  # 5 rows per CU: not taken
    for m in (2, 3, 4):  # two to four activation rows up to 12 rows per CU
        p = d.plan("rd", m, 4096, 1792, x_addr=256, w_addr=256)
        assert (p.waves, p.rows_or_rw, p.rows_per_group, p.mt, p.grid_x) == (8, 7, 7, m, 256), p
        assert d.plan("rd", m, 4096, 3584, x_addr=256, w_addr=256).rows_per_group != 14
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")
    p = d.plan("rd", 1, 4096, 1792, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.rows_per_group, p.grid_x) == (4, 4, 448), p
    monkeypatch.delenv("DMC_HIP_RD_X8")
    # ... except where one group of 8 waves per 16 rows (x in registers, a
    # window per lane) spreads evenly over at most two rounds (C1: 256 groups;
    # [8192,4096]: 512)
    for n in (4096, 8192):
        p = d.plan("rd", 1, 4096, n, x_addr=256, w_addr=256)
        assert (p.waves, p.rows_or_rw, p.rows_per_group, p.slices, p.grid_x) == (8, 4, 16, 1, n // 16), p
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")
    p = d.plan("rd", 1, 4096, 8192, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.rows_per_group, p.grid_x) == (4, 4, 2048), p
    monkeypatch.delenv("DMC_HIP_RD_X8")
    assert d.plan("rd", 1, 4096, 5120, x_addr=256, w_addr=256).rows_per_group == 4  # 320 groups: uneven
    # 1024 < K <= 2048: the same group on 4 waves (TP = 8 down share, [4096,2048]); at K = 1024 half
    # its lanes would idle; at 2 to 4 rows only on full windows from two rounds
    for k in (1792, 2048):
        p = d.plan("rd", 1, k, 4096, x_addr=256, w_addr=256)
        assert (p.waves, p.rows_or_rw, p.rows_per_group, p.grid_x) == (4, 4, 16, 256), p
    assert d.plan("rd", 1, 1024, 4096, x_addr=256, w_addr=256).rows_per_group == 4
    p = d.plan("rd", 3, 2048, 8192, x_addr=256, w_addr=256)
    assert (p.waves, p.rows_or_rw, p.rows_per_group, p.mt, p.grid_x) == (4, 4, 16, 3, 512), p
    assert d.plan("rd", 2, 2048, 4096, x_addr=256, w_addr=256).rows_per_group != 16   # one round
    assert d.plan("rd", 2, 1792, 8192, x_addr=256, w_addr=256).rows_per_group != 16   # windows not full
    p = d.plan("rd", 1, 4096, 11008, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.rows_per_group) == (2, 4), p
    # M = 1: the streaming kernel
    p = d.plan("rd", 1, 4096, 128256, x_addr=256, w_addr=256)
    assert p.mt == 1 and p.slices >= 1, p
    # M = 2 on rows of 2048 < K <= 4096: the 8-wave group (16 rows, x in
    # registers) from 3/4 of a round of groups; otherwise the streaming
    # kernel, 16 weight rows per workgroup where the grid keeps 4 workgroups
    # per CU (8 on C2 up/gate); rows16 where rows too long for the streaming
    # kernel's registers would take one activation row per pass
    for n in (128256, 14336, 4096):
        p = d.plan("rd", 2, 4096, n, x_addr=256, w_addr=256)
        assert (p.waves, p.rows_or_rw, p.slices, p.mt, p.rows_per_group, p.grid_x) == \
            (8, 4, 1, 2, 16, n // 16), p
    p = d.plan("rd", 2, 4096, 3072, x_addr=256, w_addr=256)  # 12 rows per CU: one group each
    assert (p.waves, p.rows_or_rw, p.slices, p.mt, p.rows_per_group, p.grid_x) == (8, 6, 1, 2, 12, 256), p
    assert d.plan("rd", 2, 4096, 1280, x_addr=256, w_addr=256).rows_or_rw == 2  # 80 groups of 16: streaming
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")
    p = d.plan("rd", 2, 4096, 128256, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.grid_x) == (1, 2, 16, 8016), p
    p = d.plan("rd", 2, 4096, 14336, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.grid_x) == (1, 2, 8, 1792), p
    monkeypatch.delenv("DMC_HIP_RD_X8")
    # long rows at M = 2: the 14-wave shared-x kernel with one LDS copy of x per
    # activation row (DMC_HIP_RD_X14_M2=0: the streaming kernel)
    p = d.plan("rd", 2, 14336, 4096, x_addr=256, w_addr=256)
    assert (p.waves, p.slices, p.mt, p.rows_per_group, p.grid_x) == (14, 2, 2, 16, 256), p
    monkeypatch.setenv("DMC_HIP_RD_X14_M2", "0")
    p = d.plan("rd", 2, 14336, 4096, x_addr=256, w_addr=256)
    assert (p.waves, p.mt) == (8, 2), p
    monkeypatch.delenv("DMC_HIP_RD_X14_M2")
    assert d.plan("rd", 2, 28672, 32768, x_addr=256, w_addr=256).slices == -7
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "3")
    p = d.plan("rd", 2, 28672, 32768, x_addr=256, w_addr=256)
    assert (p.slices, p.mt) == (7, 1), p   # the streaming kernel, one activation row per pass
    monkeypatch.delenv("DMC_HIP_RD_MFMA_MIN_M")
    # M >= 3 with k % 64 == 0: an MFMA kernel (slices == -kind).  M <= 4: rows16
    # (two 16-row blocks per workgroup, 4 activation rows); 6..16 rows on the LM
    # head: the gemm layout with 16-row tiles, x split in the kernel, k in one
    # slice (no workspace).  At K <= 4096 the 8-wave group takes 3 rows
    # everywhere and 4 outside one to two rounds of groups (C4: 8016).
    for m in (3, 4):
        p = d.plan("rd", m, 4096, 128256, x_addr=256, w_addr=256)
        assert (p.waves, p.rows_or_rw, p.slices, p.mt, p.rows_per_group, p.grid_x) == (8, 4, 1, m, 16, 8016), p
    assert d.plan("rd", 4, 4096, 14336, x_addr=256, w_addr=256).slices == -7  # C2 up: 896 groups
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")
    for m in (3, 4):
        p = d.plan("rd", m, 4096, 128256, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-7, 4, 32, 8, 4008), p
    monkeypatch.delenv("DMC_HIP_RD_X8")
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "2")
    p = d.plan("rd", 2, 4096, 128256, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-7, 4, 32, 8, 4008), p
    monkeypatch.delenv("DMC_HIP_RD_MFMA_MIN_M")
    p = d.plan("rd", 5, 4096, 128256, x_addr=256, w_addr=256)  # two 16-row blocks per workgroup
    assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-7, 8, 32, 8, 4008), p
    # 6..8 rows: the gemm layout on matrices above 256 MiB, rows16 up to 256 MiB
    assert d.plan("rd", 8, 4096, 28672, x_addr=256, w_addr=256).slices == -7
    assert d.plan("rd", 6, 14336, 14336, x_addr=256, w_addr=256).slices == -8
    for m in (6, 8, 9, 16):
        p = d.plan("rd", m, 4096, 128256, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x, p.workspace_bytes) == \
            (-8, 16, 256, 8, 501, 0), p
    # prefill-sized M: the gemm layout, 32 or 64 activation rows per workgroup
    for m, mt in ((17, 32), (32, 32), (33, 64), (128, 64), (512, 64)):
        p = d.plan("rd", m, 4096, 128256, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-8, mt, 256, 8, 501), p
    # k not a multiple of 64: back to the streaming kernel, activation rows held in
    # registers (MT * vectors-per-lane <= 8)
    assert d.plan("rd", 16, 4104, 1000, x_addr=256, w_addr=256).slices > 0
    for m, mt in [(2, 2), (3, 4)]:
        p = d.plan("rd", m, 4104, 1000, x_addr=256, w_addr=256)
        assert p.mt == mt and p.slices >= 1, p


@pytest.mark.parametrize("k,waves,kvec", [(8, 1, 1), (512, 1, 1), (520, 2, 1), (1024, 2, 1),
                                          (2048, 4, 1), (4096, 8, 1), (4160, 8, 2),
                                          (11008, 8, 3), (32768, 8, 8)])
def test_rowdot_streaming_kernel_covers_k(k, waves, kvec):
    p = d.plan("rd", 1, k, 1000, x_addr=256, w_addr=256)
    assert (p.waves, p.slices) == (waves, kvec), p
    assert waves * kvec * 512 >= k > (waves * kvec - waves) * 512 or kvec == 1


def test_rowdot_aligned_rows_with_a_short_last_block_take_the_short_tail():
    """Aligned rows whose last block of windows would hold 1..8 elements
    (k = 4104: 8) stream one block per lane plus a per-row short tail on the
    any-alignment kernel (reported with vec = 8) instead of a second, nearly
    empty block; at m >= 2 the streaming kernel keeps them."""
    p = d.plan("rd", 1, 4104, 11008, x_addr=256, w_addr=256)
    assert (p.vec, p.waves, p.slices, p.rows_or_rw, p.rows_per_group, p.grid_x) == (8, 8, 1, 2, 4, 2752), p
    assert d.plan("rd", 2, 4104, 11008, x_addr=256, w_addr=256).slices == 2
    assert d.plan("rd", 1, 4105, 1001, x_addr=256, w_addr=256).slices == 0   # 9 over: the general kernel


def test_rowdot_mfma_layouts(monkeypatch):
    # N too small for the wide layout: rows16, activation rows per workgroup 4,
    # 8 or 16 (DMC_HIP_RD_X8=0: at m = 3 the 8-wave group would take it)
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")
    for m, mt, rpw in [(3, 4, 32), (4, 4, 32), (5, 8, 32), (8, 8, 32)]:
        p = d.plan("rd", m, 4096, 16387, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == \
            (-7, mt, rpw, 8, (16387 + rpw - 1) // rpw), (m, p)
    monkeypatch.delenv("DMC_HIP_RD_X8")
    p = d.plan("rd", 3, 4096, 16387, x_addr=256, w_addr=256)
    assert (p.waves, p.rows_or_rw, p.rows_per_group, p.grid_x) == (8, 4, 16, 1025), p
    assert d.plan("rd", 4, 4096, 16387, x_addr=256, w_addr=256).slices == -7  # 1025 groups: one to two rounds
    # from 9 activation rows on a matrix above 128 MiB, and above 16 (past the
    # small-matrix rule) whatever N, the gemm layout (16 activation rows per
    # workgroup up to 16, 32 up to 32); at 32-row tiles on 4-wave workgroups
    # of 128 weight rows where 256-row tiles would number fewer than the CUs
    for m, mt in ((9, 16), (16, 16)):
        p = d.plan("rd", m, 4096, 16387, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-8, mt, 256, 8, 65), (m, p)
    p = d.plan("rd", 20, 4096, 16387, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-8, 32, 128, 4, 129), p
    p = d.plan("rd", 32, 4096, 128256, x_addr=256, w_addr=256)   # 501 tiles of 256 rows
    assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-8, 32, 256, 8, 501), p
    p = d.plan("rd", 33, 4096, 16387, x_addr=256, w_addr=256)    # 64-row tiles: 8 waves
    assert (p.slices, p.mt, p.rows_per_group, p.waves) == (-8, 64, 256, 8), p
    # ... except on a matrix under 64 MiB, where rows16 saves the gemm layout's
    # two extra launches (C1 at m = 12)
    p = d.plan("rd", 12, 4096, 4096, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group) == (-7, 16, 16), p
    # blocks per workgroup shrink while the grid would fall under 1 per CU:
    # C2 up/gate keeps two (448 workgroups), C1 (256 blocks, 32 MiB) one;
    # C2 down (256 blocks, 112 MiB) keeps two and splits k in two instead
    # (256 workgroups, the slices' partials in the workspace)
    p = d.plan("rd", 8, 4096, 14336, x_addr=256, w_addr=256)
    assert (p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == (8, 32, 448, 0), p
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")  # C1 at m = 4 otherwise takes the 8-wave group
    p = d.plan("rd", 4, 4096, 4096, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == (-7, 4, 16, 256, 0), p
    monkeypatch.delenv("DMC_HIP_RD_X8")
    p = d.plan("rd", 4, 4096, 4096, x_addr=256, w_addr=256)
    assert (p.waves, p.rows_or_rw, p.mt, p.rows_per_group, p.grid_x) == (8, 4, 4, 16, 256), p
    for m, mt in ((6, 8), (8, 8)):
        p = d.plan("rd", m, 14336, 4096, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == \
            (-7, mt, 32, 128, 2 * m * 4096 * 4), (m, p)
    # ... except three and four activation rows, which take the 14-wave
    # streaming kernel (x in registers, no workspace) unless an MFMA layout is
    # named or DMC_HIP_RD_X14_MAX_M lowers the bound
    for m in (3, 4):
        p = d.plan("rd", m, 14336, 4096, x_addr=256, w_addr=256)
        assert (p.waves, p.slices, p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == \
            (14, 2, m, 16, 256, 0), p
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "7")
    for m in (3, 4):
        p = d.plan("rd", m, 14336, 4096, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == \
            (-7, 4, 32, 128, 2 * m * 4096 * 4), (m, p)
    monkeypatch.delenv("DMC_HIP_RD_MFMA_KIND")
    monkeypatch.setenv("DMC_HIP_RD_X14_MAX_M", "3")
    assert d.plan("rd", 4, 14336, 4096, x_addr=256, w_addr=256).slices == -7
    monkeypatch.setenv("DMC_HIP_RD_X14_MAX_M", "2")
    assert d.plan("rd", 3, 14336, 4096, x_addr=256, w_addr=256).slices == -7
    monkeypatch.delenv("DMC_HIP_RD_X14_MAX_M")
    monkeypatch.setenv("DMC_HIP_RD_R16_SPLIT", "0")
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "7")
    p = d.plan("rd", 4, 14336, 4096, x_addr=256, w_addr=256)
    assert (p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == (4, 16, 256, 0), p
    monkeypatch.delenv("DMC_HIP_RD_R16_SPLIT")
    monkeypatch.delenv("DMC_HIP_RD_MFMA_KIND")
    # 9..16 activation rows on matrices up to 128 MiB: rows16 too, four blocks
    # per workgroup on a grid of >= 7/8 of the CUs (C2 up/gate: 224), two
    # where four would leave fewer ([8192,4096]: 256), or on C2 down four
    # blocks and k in four slices (64 x 4 workgroups); the gemm layout above
    # 128 MiB
    for m in (9, 12, 16):
        p = d.plan("rd", m, 4096, 14336, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == (-7, 16, 64, 224, 0), p
        p = d.plan("rd", m, 4096, 8192, x_addr=256, w_addr=256)
        assert (p.slices, p.rows_per_group, p.grid_x, p.workspace_bytes) == (-7, 32, 256, 0), p
        p = d.plan("rd", m, 14336, 4096, x_addr=256, w_addr=256)
        assert (p.slices, p.mt, p.rows_per_group, p.grid_x, p.workspace_bytes) == \
            (-7, 16, 64, 64, 4 * m * 4096 * 4), p
        assert d.plan("rd", m, 4096, 28672, x_addr=256, w_addr=256).slices == -8
    # at 16-row activation tiles the block count weighs rounds against the
    # x split: C1 at m = 64 takes four (256 workgroups, one round), [2048,2048]
    # at m = 160 two (640 workgroups, 3 rounds of 3) over four (320, 2 rounds of 5)
    p = d.plan("rd", 64, 4096, 4096, x_addr=256, w_addr=256)
    assert (p.slices, p.rows_per_group, p.grid_x, p.grid_x * 4) == (-7, 64, 64, 256), p
    p = d.plan("rd", 160, 2048, 2048, x_addr=256, w_addr=256)
    assert (p.slices, p.rows_per_group, p.grid_x) == (-7, 32, 64), p
    # above 16 rows, rows16 while the weights streamed (once per 16 rows)
    # total at most 128 MiB on a matrix up to 32 MiB, 80 MiB otherwise
    assert d.plan("rd", 64, 4096, 4096, x_addr=256, w_addr=256).slices == -7     # C1, 128 MiB
    assert d.plan("rd", 65, 4096, 4096, x_addr=256, w_addr=256).slices == -8     # 160 MiB
    assert d.plan("rd", 128, 4096, 2048, x_addr=256, w_addr=256).slices == -7
    assert d.plan("rd", 17, 4096, 8192, x_addr=256, w_addr=256).slices == -8     # 64 MiB matrix, 128 streamed
    assert d.plan("rd", 16, 4096, 16384, x_addr=256, w_addr=256).slices == -7    # 128 MiB at 16 rows
    assert d.plan("rd", 16, 4096, 16384 + 16, x_addr=256, w_addr=256).slices == -8
    # the gemm layout splits k while the grid stays within one workgroup per
    # CU: C2 up at m = 64 has 56 tiles of 256 x 64, so 4 slices of 16 chunks;
    # its 56 column blocks x 64 rows stay under 8192, so each workgroup
    # splits its own x and the workspace holds only the 4 partial sums
    p = d.plan("rd", 64, 4096, 14336, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.grid_x) == (-8, 64, 56), p
    assert p.workspace_bytes == 4 * 64 * 14336 * 4, p
    # up at m = 192: 168 tiles would leave a lone round a third empty, so
    # k splits to fill two rounds (3 slices); 56 x 192 > 8192, so x is split
    # once, by a launch, into three bf16 planes in the workspace
    p = d.plan("rd", 192, 4096, 14336, x_addr=256, w_addr=256)
    assert p.workspace_bytes == 3 * 192 * 4096 * 2 + 3 * 192 * 14336 * 4, p
    monkeypatch.setenv("DMC_HIP_GEMM_FUSE", "2")   # always split in the kernel
    assert d.plan("rd", 192, 4096, 14336, x_addr=256, w_addr=256).workspace_bytes == 3 * 192 * 14336 * 4
    monkeypatch.setenv("DMC_HIP_GEMM_FUSE", "0")   # never (planes even at 16-row tiles)
    assert d.plan("rd", 64, 4096, 14336, x_addr=256, w_addr=256).workspace_bytes == \
        3 * 64 * 4096 * 2 + 4 * 64 * 14336 * 4
    monkeypatch.delenv("DMC_HIP_GEMM_FUSE")
    # down at m = 32: 32 tiles of 128 x 32 (4-wave workgroups), 16 slices of 14 chunks
    p = d.plan("rd", 32, 14336, 4096, x_addr=256, w_addr=256)
    assert (p.mt, p.waves, p.workspace_bytes) == (32, 4, 16 * 32 * 4096 * 4), p
    p = d.plan("rd", 512, 4096, 128256, x_addr=256, w_addr=256)   # 4008 tiles: no split
    assert p.workspace_bytes == 3 * 512 * 4096 * 2, p
    # x's three bf16 planes must stay inside one buffer range (6 m k < 2^31):
    # beyond that the rows16 layout, which reads x directly
    p = d.plan("rd", 32768, 11008, 4096, x_addr=256, w_addr=256)
    assert (p.slices, p.mt) == (-7, 16), p
    p = d.plan("rd", 32512, 11008, 4096, x_addr=256, w_addr=256)  # 6 m k = 2,147,352,576 < 2^31
    assert p.slices == -8, p
    monkeypatch.setenv("DMC_HIP_RD_R16_TILES", "4")
    p = d.plan("rd", 16, 4096, 128256, x_addr=256, w_addr=256)
    assert p.slices == -8, p  # tiles only shape the rows16 layout
    p = d.plan("rd", 4, 4096, 128256, x_addr=256, w_addr=256)
    assert (p.slices, p.rows_per_group, p.grid_x) == (-7, 64, 2004), p
    monkeypatch.delenv("DMC_HIP_RD_R16_TILES")
    # either layout can be forced
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "7")
    p = d.plan("rd", 16, 4096, 128256, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.grid_x) == (-7, 16, 64, 2004), p
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "6")
    p = d.plan("rd", 16, 4096, 1000, x_addr=256, w_addr=256)
    assert (p.slices, p.rows_per_group, p.waves, p.grid_x) == (-6, 256, 8, 4), p
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "8")
    p = d.plan("rd", 4, 4096, 1000, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.grid_x) == (-8, 16, 256, 4), p
    monkeypatch.setenv("DMC_HIP_GEMM_MT", "32")
    p = d.plan("rd", 4, 4096, 1000, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-8, 32, 128, 4, 8), p
    monkeypatch.setenv("DMC_HIP_GEMM_WAVES", "8")
    p = d.plan("rd", 4, 4096, 1000, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.rows_per_group, p.waves, p.grid_x) == (-8, 32, 256, 8, 4), p
    monkeypatch.delenv("DMC_HIP_GEMM_WAVES")
    monkeypatch.delenv("DMC_HIP_GEMM_MT")
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "0")  # disabled: the FMA kernels
    assert d.plan("rd", 16, 4096, 128256, x_addr=256, w_addr=256).slices > 0


def test_rowdot_falls_back_to_general_kernel():
    # k beyond the register budget (eight windows per lane), k == 0, several
    # activation rows on misaligned weights, x not 16-byte aligned
    for m, k, x, w in [(1, 32776, 256, 256), (1, 32767, 256, 256), (1, 28681, 256, 256), (1, 0, 256, 256),
                       (2, 4097, 256, 256), (1, 4097, 260, 256), (1, 32770, 256, 258)]:
        p = d.plan("rd", m, k, 1000, x_addr=x, w_addr=w)
        assert p.slices == 0 and p.waves == 4, (m, k, x, w, p)


@pytest.mark.parametrize("k,w,waves,kvec,rows", [(6145, 256, 8, 2, 1), (4096, 258, 8, 1, 2), (11007, 256, 8, 3, 2),
                                                 (1023, 256, 2, 1, 2), (257, 256, 1, 1, 2), (16384, 262, 8, 4, 2),
                                                 (28671, 256, 8, 7, 1), (4095, 256, 8, 1, 2)])
def test_rowdot_misaligned_rows_stream_unaligned(k, w, waves, kvec, rows):
    """Rows that do not start on 16-byte boundaries (odd k, an offset
    weight) at m = 1: the streaming layout with unaligned 128-bit loads,
    reported as a streaming plan (slices > 0) with vec < 8.  With n odd the
    matrix's last element ends on a dword boundary, so no padding is needed."""
    p = d.plan("rd", 1, k, 11007, x_addr=256, w_addr=w)
    assert p.vec < 8 and (p.waves, p.slices, p.rows_or_rw, p.mt) == (waves, kvec, rows, 1), p
    assert p.grid_x * p.rows_per_group >= 11007


def test_rowdot_unaligned_reads_whole_dwords_only():
    """The any-alignment kernel reads every row from the dword boundary at or
    below its start, so the dword holding the matrix's last element always
    lies inside the descriptor (odd k with n even puts that element at 2 mod
    4: it still streams).  With ldw odd the rows alternate between 0 and 2
    mod 4, and each workgroup takes every other row of a block of 2 * rpw."""
    for n in (11008, 11007):
        p = d.plan("rd", 1, 4095, n, x_addr=256, w_addr=256)
        assert (p.vec, p.slices, p.rows_per_group) == (1, 1, 4), p
        assert p.grid_x == 2 * ((n + 7) // 8), p
    p = d.plan("rd", 1, 4096, 11008, x_addr=256, w_addr=258)   # k even, W at 2 mod 4: every row shifted
    assert (p.vec, p.slices, p.grid_x) == (1, 1, 2752), p


def test_rowdot_unaligned_needs_a_well_filled_last_block_or_a_short_tail():
    """Misaligned rows stay on the streaming kernel when the last block of
    windows is at least half full (k = 4095), or when 1..8 elements are left
    past whole blocks (k = 4097, 8199: a per-row short tail, read element by
    element, so no padding behind the matrix is needed); a last block holding
    9 to 2047 elements goes to the general kernel (k = 4105), as does a
    single block less than half full (k = 7)."""
    p = d.plan("rd", 1, 4097, 11007, x_addr=256, w_addr=256)
    assert (p.slices, p.waves, p.rows_per_group) == (1, 8, 4), p
    assert d.plan("rd", 1, 8199, 4097, x_addr=256, w_addr=256).slices == 2
    assert d.plan("rd", 1, 4095, 11008, x_addr=256, w_addr=258).slices == 1  # last element at 0 mod 4
    assert d.plan("rd", 1, 4105, 11007, x_addr=256, w_addr=256).slices == 0
    assert d.plan("rd", 1, 7, 1001, x_addr=256, w_addr=256).slices == 0
    monkey = os.environ.get("DMC_HIP_RD_SHORT_TAIL")
    os.environ["DMC_HIP_RD_SHORT_TAIL"] = "0"
    try:
        assert d.plan("rd", 1, 4097, 11007, x_addr=256, w_addr=256).slices == 0
    finally:
        if monkey is None:
            del os.environ["DMC_HIP_RD_SHORT_TAIL"]
        else:
            os.environ["DMC_HIP_RD_SHORT_TAIL"] = monkey


def test_column_stream_plans_split_k_and_size_workspace():
    # streaming kernel: 512 columns per workgroup, k split so ~2 workgroups per
    # CU with at most 16 column blocks (C2 down: 8), ~4 with more (C2 up: 28)
    p = d.plan("cs", 1, 14336, 4096, x_addr=256, w_addr=256)
    assert p.vec == 8 and p.waves == 4 and p.grid_x == 8 and p.slices > 1
    assert p.workspace_bytes == p.slices * 4096 * 4
    assert 512 - p.grid_x <= p.grid_x * p.slices <= 512 + p.grid_x, p
    assert p.rows_per_group * p.slices >= 14336 > p.rows_per_group * (p.slices - 1)
    up = d.plan("cs", 1, 4096, 14336, x_addr=256, w_addr=256)
    assert up.grid_x == 28 and up.rows_per_group % 4 == 0
    assert 1024 - up.grid_x <= up.grid_x * up.slices <= 1024 + up.grid_x, up
    one = d.plan("cs", 1, 32, 4096, x_addr=256, w_addr=256)  # >= 8 k rows per wave
    assert one.slices == 1 and one.workspace_bytes == 0
    assert d.plan("cs", 16, 4096, 4096, x_addr=256, w_addr=256).mt == 4
    assert p.rows_or_rw == 0 and up.rows_or_rw == 0  # the streaming kernel
    # N not a multiple of 8: the streaming kernel over misaligned rows, the
    # last k row left to the slice pass (which needs its workspace even for
    # one slice); tiny N or K = 1: the general kernel
    odd = d.plan("cs", 1, 4097, 11007, x_addr=256, w_addr=256)
    assert (odd.vec, odd.rows_or_rw, odd.waves) == (1, 0, 4), odd
    assert odd.rows_per_group * odd.slices >= 4096 > odd.rows_per_group * (odd.slices - 1)
    assert odd.workspace_bytes == odd.slices * 11007 * 4
    c5 = d.plan("cs", 1, 11008, 4097, x_addr=256, w_addr=256)
    assert (c5.vec, c5.rows_or_rw) == (1, 0) and c5.workspace_bytes == c5.slices * 4097 * 4, c5
    view = d.plan("cs", 1, 4096, 14336, x_addr=256, w_addr=258)  # a view 2 bytes into its region
    assert (view.vec, view.rows_or_rw) == (1, 0), view
    for k, n in [(1, 4097), (64, 7)]:
        g = d.plan("cs", 1, k, n, x_addr=256, w_addr=256)
        assert g.rows_or_rw > 0, (k, n, g)
    zero_k = d.plan("cs", 1, 0, 512, x_addr=256, w_addr=256)
    assert zero_k.slices == 1


def test_column_stream_row_groups_for_narrow_n(monkeypatch):
    """Narrow N on the streaming kernel (batched per-head projections): G row
    groups per wave over 512/G columns, the fewest groups whose columns cover
    N, reported as rows_or_rw = -G (0 for one group; > 0 is the general
    kernel); 4 waves only, aligned rows."""
    for n, g in ((8, 8), (64, 8), (72, 4), (128, 4), (136, 2), (256, 2), (264, 0), (512, 0), (4096, 0)):
        p = d.plan("cs", 1, 4096, n, batch=32, rs=4096 * n, x_addr=256, w_addr=256)
        assert (p.vec, p.waves, p.rows_or_rw, p.grid_x) == (8, 4, -g, -(-n // (512 // max(g, 1)))), (n, p)
        assert p.workspace_bytes == (p.slices * 32 * n * 4 if p.slices > 1 else 0), (n, p)
    monkeypatch.setenv("DMC_HIP_CS_WAVES", "8")        # row groups only at 4 waves
    assert d.plan("cs", 1, 4096, 128, batch=32, rs=4096 * 128, x_addr=256, w_addr=256).rows_or_rw == 0
    monkeypatch.delenv("DMC_HIP_CS_WAVES")
    monkeypatch.setenv("DMC_HIP_CS_ROW_GROUPS", "8")   # forced on a wide N: 64 columns per workgroup
    p = d.plan("cs", 1, 2048, 1024, batch=2, rs=2048 * 1024, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.grid_x) == (-8, 16), p
    p = d.plan("cs", 1, 4096, 4097, x_addr=256, w_addr=256)  # odd N: misaligned rows, one group
    assert (p.vec, p.rows_or_rw) == (1, 0), p


# ---- errors without a device ------------------------------------------------------------------

def test_int_entries_reject_bad_shapes_before_touching_a_device():
    lib = _lib.load()
    assert lib.dmc_hip_gemv_rd(0, 0, 0, -1, 4, 4) == -2
    assert lib.dmc_hip_gemv_cs(0, 0, 0, 1, 4, 4, -1, 0, 0) == -2
    assert lib.dmc_hip_gemv_rd(0, 0, 0, 1, 1 << 31, 4) == -2
    assert lib.dmc_hip_region_alloc(0) == 0
    assert b"positive" in lib.dmc_hip_last_error()
    assert lib.dmc_hip_gemv_rd(0, 0, 0, 0, 4, 4) == 0  # m == 0: no-op, no device needed


def test_python_api_validates_before_calling():
    with pytest.raises(TypeError):
        d.matmul_bf16_gpu(np.ones((1, 4), np.float64), np.ones((4, 2), np.uint16))
    with pytest.raises(ValueError):
        d.matmul_bf16_gpu(np.ones((1, 4), np.float32), np.ones((5, 2), np.uint16))
    with pytest.raises(ValueError):
        d.matmul_bf16_gpu_t(np.ones((1, 4), np.float32), np.ones((2, 5), np.uint16))
    with pytest.raises(ValueError):
        d.matmul_bf16_gpu_batched(np.ones(4, np.float32), np.ones(8, np.uint16), 1, 4, 2, 3, 4, 8)


def _run_isolated(code: str, **env):
    e = dict(os.environ)
    e.update(env)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=e,
                          cwd=str(ROOT), timeout=120)


def test_unavailable_when_disabled():
    r = _run_isolated("import demonic_amd as d; print(d.available()); "
                      "print(d._lib.load().dmc_hip_last_error().decode())", DMC_HIP_DISABLE="1")
    assert r.returncode == 0, r.stderr
    assert r.stdout.split("\n")[0] == "False"
    assert "DMC_HIP_DISABLE" in r.stdout


def test_dropin_entry_fails_loudly_without_a_device():
    """No CPU fallback: with the device unavailable the void entry aborts with
    a message instead of writing anything (callers ask dmc_hip_available first)."""
    code = ("import numpy as np, demonic_amd as d\n"
            "x = np.ones((1, 8), np.float32); w = np.ones((8, 4), np.uint16)\n"
            "d.matmul_bf16_gpu(x, w)\nprint('returned')\n")
    r = _run_isolated(code, DMC_HIP_DISABLE="1")
    assert r.returncode != 0
    assert "dmc_hip: fatal: dmc_matmul_bf16_gpu" in r.stderr
    assert "returned" not in r.stdout


def test_flush_before_first_use_is_a_noop():
    r = _run_isolated("import demonic_amd as d; d.flush(); print('ok')", DMC_HIP_DISABLE="1")
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr


def test_package_has_no_cpu_gemv_and_never_imports_the_oracle():
    src = "\n".join(p.read_text() for p in (ROOT / "demonic_amd").rglob("*.py"))
    src += "\n".join(p.read_text() for p in (ROOT / "demonic_amd" / "csrc").glob("*"))
    assert "import oracle" not in src and "from oracle" not in src
    assert "fmaf(" not in (ROOT / "demonic_amd" / "csrc" / "dmc_hip_runtime.cpp").read_text()


# ---- the f32 route (jit.rs:20806-20831) -----------------------------------------------------

def test_f32_selection_predicate():
    sel = d.f32_selected
    assert sel(True, 0, 4096, 4096, 1), "W @ x refused"
    assert sel(True, 0, 1, 4096, 4096), "x @ W refused"
    assert sel(True, 0, 16, 4096, 4096) and sel(True, 0, 4096, 4096, 16)
    assert not sel(True, 0, 17, 4096, 17), "a GEMM shape selected"
    assert not sel(False, 0, 4096, 4096, 1) and not sel(True, 1, 4096, 4096, 1)
    assert not sel(True, 0, 64, 128, 1), "small GEMV selected"
    assert not sel(True, 0, 0, 4096, 1) and not sel(True, 0, 4096, 0, 1)


@pytest.mark.parametrize("k,waves,kvec,rows", [(4, 1, 1, 2), (256, 1, 1, 2), (1000, 4, 1, 2), (2048, 8, 1, 2),
                                               (4096, 8, 2, 2), (6144, 8, 3, 1), (14336, 8, 7, 1),
                                               (16384, 8, 8, 1)])
def test_f32_streaming_plan_covers_k(k, waves, kvec, rows):
    p = d.plan_f32(1, k, 14336, x_addr=256, w_addr=256)
    assert (p.waves, p.kvec, p.rows) == (waves, kvec, rows), p
    assert kvec * waves * 256 >= k > (kvec - 1) * waves * 256 or kvec == 1
    assert p.grid_x * p.rows_per_group >= 14336 and p.rows_per_group % p.rows == 0


@pytest.mark.parametrize("k,x_addr,w_addr", [(4097, 256, 256), (4098, 256, 256), (16388, 256, 256),
                                             (4096, 260, 256), (4096, 256, 264)])
def test_f32_general_kernel_for_odd_k_misaligned_or_long_rows(k, x_addr, w_addr):
    p = d.plan_f32(1, k, 14336, x_addr=x_addr, w_addr=w_addr)
    assert p.kvec == 0 and p.waves == 4 and p.rows_per_group == 4 and p.grid_x == 14336 // 4, p


def test_f32_activation_rows_per_workgroup(monkeypatch):
    assert d.plan_f32(4, 4096, 4096, x_addr=256, w_addr=256).mt == 4      # kvec 2: up to 4
    # 2048 < K <= 4096: the 8-wave group (16 rows, two windows per lane) at 3 and 4 rows, and
    # where K is not a multiple of 2048; the streaming kernel (4 rows per workgroup) otherwise
    for m, k, group in ((3, 4096, True), (4, 4096, True), (1, 4096, False), (2, 4096, False), (1, 3072, True),
                        (2, 2560, True), (4, 2048, False)):
        p = d.plan_f32(m, k, 4096, x_addr=256, w_addr=256)
        assert (p.waves == 8 and p.rows_per_group == 16) == group, (m, k, p)
        if group:
            assert (p.kvec, p.mt, p.grid_x, p.grid_y) == (2, m, 256, 1), p
    monkeypatch.setenv("DMC_HIP_F32_X8", "0")
    assert d.plan_f32(4, 4096, 4096, x_addr=256, w_addr=256).rows_per_group == 4
    monkeypatch.delenv("DMC_HIP_F32_X8")
    assert d.plan_f32(16, 4096, 4096, x_addr=256, w_addr=256).grid_y == 4
    # long rows that the 8-wave kernel would take one activation row per pass
    # (kvec 7 at K = 14336): the 14-wave kernel, every activation row in one
    # pass; a lone row, and a grid short of one 16-row workgroup per CU, keep
    # the 8-wave kernel (DMC_HIP_F32_X14=2 takes the 14-wave one there too)
    for m in (2, 3, 4):
        p = d.plan_f32(m, 14336, 4096, x_addr=256, w_addr=256)
        assert (p.waves, p.kvec, p.mt, p.rows_per_group, p.grid_x, p.grid_y) == (14, 4, m, 16, 256, 1), p
    assert d.plan_f32(1, 14336, 4096, x_addr=256, w_addr=256).waves == 8
    assert d.plan_f32(2, 8192, 4096, x_addr=256, w_addr=256).waves == 8   # kvec 4: two per pass
    assert d.plan_f32(3, 8192, 4096, x_addr=256, w_addr=256).waves == 14
    assert d.plan_f32(2, 14336, 1000, x_addr=256, w_addr=256).waves == 8
    monkeypatch.setenv("DMC_HIP_F32_X14", "0")
    assert d.plan_f32(4, 14336, 4096, x_addr=256, w_addr=256).mt == 1     # kvec 7: one
    monkeypatch.setenv("DMC_HIP_F32_X14", "2")
    assert d.plan_f32(1, 14336, 1000, x_addr=256, w_addr=256).waves == 14
    monkeypatch.delenv("DMC_HIP_F32_X14")
    assert d.plan_f32(16, 4097, 64, x_addr=256, w_addr=256).mt == 16      # general


def test_f32_entries_reject_gemm_shapes_before_touching_a_device():
    lib = _lib.load()
    l = np.ones((17, 8), np.float32)
    r = np.ones((8, 17), np.float32)
    out = np.full((17, 17), 7.0, np.float32)
    assert lib.dmc_matmul_f32_gpu_try(l.ctypes.data, r.ctypes.data, out.ctypes.data, 17, 8, 17) == -2
    assert b"GEMV shapes only" in lib.dmc_hip_last_error()
    assert np.all(out == 7.0)
    assert lib.dmc_matmul_f32_gpu_try(0, 0, out.ctypes.data, 1, 8, -1) == -2
    assert lib.dmc_matmul_f32_gpu_try(0, 0, out.ctypes.data, 0, 8, 4) == 0  # m == 0: no-op
    assert lib.dmc_hip_gemv_f32_rd(0, 0, 0, -1, 4, 4) == -2


def test_f32_dropin_fails_loudly_without_a_device():
    code = ("import numpy as np, demonic_amd as d\n"
            "print(d.matmul_f32_gpu_try(np.ones((4, 8), np.float32), np.ones(8, np.float32))[0], flush=True)\n"
            "d.matmul_f32_gpu(np.ones((4, 8), np.float32), np.ones(8, np.float32))\nprint('returned')\n")
    r = _run_isolated(code, DMC_HIP_DISABLE="1")
    assert r.returncode != 0
    assert r.stdout.split("\n")[0] == "-1"  # DMC_HIP_ENODEV from the try form
    assert "dmc_hip: fatal: dmc_matmul_f32_gpu" in r.stderr
    assert "returned" not in r.stdout


def test_gemm_layout_with_fused_split_and_one_slice_has_no_workspace():
    """m = 9..16 on 65k-98k rows: the tiles fill the device, so the gemm layout
    keeps k in one slice and splits x itself -- no workspace (the launch is
    then given none)."""
    p = d.plan("rd", 12, 1024, 80000, x_addr=256, w_addr=256)
    assert (p.slices, p.mt, p.workspace_bytes, p.grid_x) == (-8, 16, 0, 313), p
