"""Instruction-order checks on the gfx950 assembly of kernels whose
synchronisation depends on it (CPU only: hipcc cross-compiles here): the
M = 1 GEMVs' copy-then-wait order, scalar LDS addresses for every
direct-to-LDS copy, and the issue order the two-half copies of the M = 9..16
MFMA tile GEMVs wait on.

gemv_q4_0_m1_kernel<true> and gemv_q4_K_kernel<1, true, false> copy the activation
row into LDS with direct loads (global_load_lds_*) and then issue the loads
of each lane's first weight step before waiting; the wait before the
workgroup barrier is `s_waitcnt vmcnt(3)`, which covers the copies only
because vector-memory loads complete in issue order and at least three
weight loads were issued after the last copy on every path. If the compiler
ever moved those weight loads below the wait (into a branch, say), vmcnt(3)
would no longer wait for the copies and waves could read LDS before it is
filled; this test fails instead.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "qgemm-perf-framework-ng_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _kernel_lines(asm: str, symbol_part: str) -> list[str]:
    """Instruction and label lines of the first function whose label contains symbol_part."""
    lines = [ln.split(";")[0].strip() for ln in asm.splitlines()]
    start = next(i for i, ln in enumerate(lines) if ln.endswith(":") and symbol_part in ln and not ln.startswith("."))
    out = []
    for t in lines[start + 1:]:
        if not t or (t.startswith(".") and not t.endswith(":")):
            continue
        out.append(t)
        if t.startswith("s_endpgm"):
            break
    return out


def check_copy_then_wait(lines: list[str], min_loads: int = 3) -> None:
    """The order the vmcnt(3) wait needs (raises AssertionError otherwise)."""
    wait = next(i for i in range(len(lines) - 1)
                if lines[i] == "s_waitcnt vmcnt(3)" and lines[i + 1] == "s_barrier")
    dma = [i for i, t in enumerate(lines) if t.startswith("global_load_lds")]
    assert dma, "no direct-to-LDS copy found"
    assert max(dma) < wait, "a direct-to-LDS copy is issued after the wait"
    # straight-line stretch that every path to the wait runs through
    labels = [i for i in range(wait) if lines[i].endswith(":")]
    first = labels[-1] + 1 if labels else 0
    assert first > max(dma), "a path to the wait may skip the weight loads"
    seg = lines[first:wait]
    assert not any(re.match(r"s_(c)?branch", t) for t in seg), "branch between the copies and the wait"
    loads = [t for t in seg if re.match(r"(global|buffer)_load_(?!lds)", t)]
    assert len(loads) >= min_loads, f"only {len(loads)} weight loads between the copies and vmcnt(3)"
    # a shorter wait before the barrier (weights decoded above it) would be
    # correct but would make every wave wait for its weights there
    for t in seg:
        m = re.match(r"s_waitcnt .*vmcnt\((\d+)\)", t)
        assert not (m and int(m.group(1)) < 3), f"early weight wait before the barrier: {t}"


def test_checker_rejects_sunk_loads():
    """The checker itself: loads moved below the wait must fail it."""
    good = ["global_load_lds_dwordx4 v[0:1], off", ".LBB0_2:", "global_load_dwordx4 v[0:3], v9, s[4:5]",
            "global_load_dword v4, v9, s[4:5] offset:32", "global_load_dwordx4 v[5:8], v9, s[4:5] offset:16",
            "s_waitcnt vmcnt(3)", "s_barrier", "ds_read_b32 v1, v2", "s_endpgm"]
    check_copy_then_wait(good)
    sunk = good[:2] + ["s_waitcnt vmcnt(3)", "s_barrier"] + good[2:5] + good[7:]
    with pytest.raises(AssertionError):
        check_copy_then_wait(sunk)
    branchy = good[:2] + ["s_cbranch_execz .LBB0_3"] + good[2:]
    with pytest.raises(AssertionError):
        check_copy_then_wait(branchy)
    early = good[:5] + ["s_waitcnt vmcnt(0)", "v_and_b32_e32 v1, 15, v2"] + good[5:]
    with pytest.raises(AssertionError):
        check_copy_then_wait(early)


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None, reason="needs hipcc and make")
@pytest.mark.parametrize("source,kernel", [("gemv.hip", "gemv_q4_0_m1_kernelILb1E"),
                                           ("gemv_kquant.hip", "gemv_q4_K_kernelILi1ELb1ELb0E")])
def test_m1_gemv_copy_precedes_wait(source, kernel):
    out = os.path.join(PKG_DIR, "_build", source + ".s")
    subprocess.run(["make", "-s", "-C", PKG_DIR, out], check=True, capture_output=True, timeout=600)
    with open(out) as f:
        asm = f.read()
    check_copy_then_wait(_kernel_lines(asm, kernel))


def dma_m0_from_vector(lines: list[str]) -> list[str]:
    """Direct-to-LDS loads whose LDS address (M0) was set from a
    v_readfirstlane of a vector register: the compiler does this when it merges
    copy sites of divergent paths into one, and lanes of the other path then
    write to the first active lane's address."""
    bad, rfl = [], {}
    for i, t in enumerate(lines):
        m = re.match(r"s_mov_b32 m0, (s\d+)", t)
        if m and m.group(1) in rfl and any("load_lds" in u for u in lines[i:i + 6]):
            bad.append(f"{rfl[m.group(1)]} -> {t}")
        # a scalar register redefined by any other instruction no longer
        # holds the read-first-lane value
        d = re.match(r"\S+\s+s(?:\[(\d+):(\d+)\]|(\d+)\b)", t)
        if d:
            lo = int(d.group(1) or d.group(3))
            hi = int(d.group(2) or d.group(3))
            for r in range(lo, hi + 1):
                rfl.pop(f"s{r}", None)
        m = re.match(r"v_readfirstlane_b32 (s\d+),", t)
        if m:
            rfl[m.group(1)] = t
    return bad


def test_dma_checker_flags_vector_m0():
    """The checker itself: an M0 taken from a readfirstlane before a copy."""
    good = ["s_add_i32 m0, s21, 0x400", "global_load_lds_dwordx4 v[2:3], off"]
    assert dma_m0_from_vector(good) == []
    bad = ["v_add_u32_e32 v1, s21, v10", "v_readfirstlane_b32 s0, v1", "s_mov_b32 m0, s0",
           "global_load_lds_dwordx4 v[6:7], off"]
    assert dma_m0_from_vector(bad)
    # the wave index read from lane 0, then the register reused for a scalar base
    reused = ["v_readfirstlane_b32 s14, v0", "s_lshr_b32 s13, s14, 6", "s_add_i32 s14, s13, 0x400",
              "s_mov_b32 m0, s14", "global_load_lds_dwordx4 v[2:3], off"]
    assert dma_m0_from_vector(reused) == []
    pair = ["v_readfirstlane_b32 s15, v3", "s_load_dwordx2 s[14:15], s[0:1], 0x0", "s_mov_b32 m0, s15",
            "global_load_lds_dwordx4 v[2:3], off"]
    assert dma_m0_from_vector(pair) == []


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None, reason="needs hipcc and make")
@pytest.mark.parametrize("source", ["gemv.hip", "gemv_kquant.hip", "gemm_small.hip"])
def test_dma_lds_address_is_scalar(source):
    """Every direct-to-LDS copy in the kernels that use them takes its LDS
    address from scalar code (a workgroup- or wave-uniform base)."""
    out = os.path.join(PKG_DIR, "_build", source + ".s")
    subprocess.run(["make", "-s", "-C", PKG_DIR, out], check=True, capture_output=True, timeout=600)
    with open(out) as f:
        lines = [ln.split(";")[0].strip() for ln in f.read().splitlines()]
    assert dma_m0_from_vector(lines) == []


def check_half_split(lines: list[str], copies: int, after_half0: int, lead: int = 0) -> None:
    """Two-half copies (the iq2_xxs M = 5..8 MFMA tile GEMV): the wave's run of
    `copies` direct-to-LDS instructions writes consecutive 1-KB pieces of its
    LDS region in issue order (M0 = base + 0x400 i), and the first wait after
    the run is vmcnt(after_half0): loads complete in issue order, so it holds
    the wave until the instructions that wrote half 0 have landed. A run
    reordered by the compiler would make that wait cover the wrong pieces.
    `lead` copies into the same region (the wave's own table pieces, issued
    before the run) are dropped first; they must precede the run."""
    run, m0 = [], None
    for i, t in enumerate(lines):
        m = re.match(r"s_mov_b32 m0, (s\d+)$", t)
        if m:
            m0 = (m.group(1), 0)
        m = re.match(r"s_add_i32 m0, (s\d+), (0x[0-9a-f]+|\d+)$", t)
        if m:
            m0 = (m.group(1), int(m.group(2), 0))
        elif t.startswith("s_add_i32 m0,"):
            m0 = None  # a base plus a register: not part of the run (a table piece)
        if t.startswith("global_load_lds") and m0 is not None:
            run.append((i, m0))
    assert len(run) == copies + lead, f"{len(run)} copies, expected {lead} + {copies}"
    run = run[lead:]
    assert len({b for _, (b, _) in run}) == 1, "the run's copies use different LDS bases"
    offsets = [o for _, (_, o) in run]
    assert offsets == [0x400 * (offsets[0] // 0x400 + k) for k in range(copies)], f"run out of order: {offsets}"
    waits = [t for t in lines[run[-1][0]:] if re.match(r"s_waitcnt .*vmcnt\(\d+\)", t)]
    run_wait = next(t for t in waits if int(re.search(r"vmcnt\((\d+)\)", t).group(1)) < copies)
    assert f"vmcnt({after_half0})" in run_wait, f"first wait on the run is {run_wait}"


def test_half_split_checker():
    """The checker itself: a swapped pair of copies or a wrong wait fails."""
    good = ["s_mov_b32 m0, s14", "global_load_lds_dwordx4 v[2:3], off", "s_add_i32 m0, s14, 0x400",
            "global_load_lds_dwordx4 v[2:3], off", "s_add_i32 m0, s14, 0x800", "global_load_lds_dwordx4 v2, s[4:5]",
            "s_waitcnt vmcnt(1)", "ds_read_b32 v1, v2", "s_waitcnt vmcnt(0)", "s_endpgm"]
    check_half_split(good, 3, 1)
    swapped = good[:2] + good[4:6] + good[2:4] + good[6:]
    with pytest.raises(AssertionError):
        check_half_split(swapped, 3, 1)
    with pytest.raises(AssertionError):
        check_half_split(good, 3, 2)
    table = ["s_add_i32 m0, s14, s8", "global_load_lds_dwordx4 v1, s[8:9]"] + good[:6] + ["s_waitcnt vmcnt(3)"] + good[6:]
    check_half_split(table, 3, 1)
    # two leading pieces into the same region, then the run at 0x800..
    lead = ["s_mov_b32 m0, s14", "global_load_lds_dwordx4 v1, s[8:9]", "s_add_i32 m0, s14, 0x400",
            "global_load_lds_dwordx4 v1, s[8:9]"]
    run3 = lead + ["s_add_i32 m0, s14, 0x800", good[1], "s_add_i32 m0, s14, 0xc00", good[3],
                   "s_add_i32 m0, s14, 0x1000", good[5]] + good[6:]
    check_half_split(run3, 3, 1, lead=2)
    with pytest.raises(AssertionError):  # the leading pieces not declared
        check_half_split(run3, 3, 1)


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None, reason="needs hipcc and make")
@pytest.mark.parametrize("source,kernel,copies,after_half0,lead", [
    ("gemv_kquant.hip", "gemv_iq2_xxs_mfma_sb_kernelILi5E", 3, 1, 0),
    ("gemv_kquant.hip", "gemv_iq2_xxs_mfma_sb_kernelILi8E", 4, 2, 3),  # its own three table pieces first
])
def test_half_split_copy_order(source, kernel, copies, after_half0, lead):
    out = os.path.join(PKG_DIR, "_build", source + ".s")
    subprocess.run(["make", "-s", "-C", PKG_DIR, out], check=True, capture_output=True, timeout=600)
    with open(out) as f:
        asm = f.read()
    check_half_split(_kernel_lines(asm, kernel), copies, after_half0, lead)


def check_chunk_waits(lines: list[str], chunks: int, table_wait: int | None = None) -> None:
    """The chunked MFMA tile GEMVs (from k = 4096, up to m = 128): no scratch memory
    (spill loads and stores would count in vmcnt and break the waits'
    arithmetic), and the vector-memory waits are exactly the designed ones: one
    vmcnt(3) before each half of each chunk but the last, which waits for
    everything. A kernel with a table wait (table_wait: its vmcnt) has it
    exactly once; it may be laid out after the loop body, so only its count is
    checked. (The iq2_xxs kernel has none: each wave's own table copy goes out
    before its first weight copy, so the first vmcnt(3) covers it.)"""
    assert not any(t.startswith("scratch_") or "buffer_store" in t for t in lines), "register spills"
    waits = [int(re.search(r"vmcnt\((\d+)\)", t).group(1)) for t in lines if re.match(r"s_waitcnt .*vmcnt", t)]
    if table_wait is not None:
        assert waits.count(table_wait) == 1, f"waits {waits}: expected one table wait vmcnt({table_wait})"
        waits.remove(table_wait)
    expect = [3] * (2 * chunks - 1) + [0]
    assert waits[:len(expect)] == expect, f"waits {waits}, expected to start {expect}"


def test_chunk_wait_checker():
    lines = ["global_load_lds_dwordx4 v[2:3], off", "s_waitcnt vmcnt(3)", "ds_read_b32 v1, v2", "s_waitcnt vmcnt(3)",
             "s_waitcnt vmcnt(3)", "s_waitcnt vmcnt(0)", "s_barrier"]
    check_chunk_waits(lines, 2)
    with pytest.raises(AssertionError):  # an extra full wait inside the chunks
        check_chunk_waits(lines[:2] + ["s_waitcnt vmcnt(0)"] + lines[2:], 2)
    with pytest.raises(AssertionError):
        check_chunk_waits(lines[:2] + ["scratch_store_dword off, v1, off"] + lines[2:], 2)
    table = lines + ["s_waitcnt vmcnt(8)", "s_barrier"]  # the table wait laid out after the loop
    check_chunk_waits(table, 2, 8)
    with pytest.raises(AssertionError):  # no table wait
        check_chunk_waits(lines, 2, 8)
    with pytest.raises(AssertionError):  # two
        check_chunk_waits(["s_waitcnt vmcnt(8)"] + table, 2, 8)


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None, reason="needs hipcc and make")
@pytest.mark.parametrize("source,kernel,table_wait", [("gemv.hip", "gemv_q4_0_mfma_chunk_kernel", None),
                                                      ("gemv_kquant.hip", "gemv_q4_K_mfma_chunk_kernel", None),
                                                      ("gemv_kquant.hip", "gemv_iq2_xxs_mfma_chunk_kernel", None)])
@pytest.mark.parametrize("chunks", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("groups", [0, 16])
def test_chunked_gemv_waits(source, kernel, table_wait, chunks, groups):
    """Both forms: the group count read at run time (0, any number of rounds) and
    fixed at 16 (k = 4096, one round)."""
    out = os.path.join(PKG_DIR, "_build", source + ".s")
    subprocess.run(["make", "-s", "-C", PKG_DIR, out], check=True, capture_output=True, timeout=600)
    with open(out) as f:
        asm = f.read()
    check_chunk_waits(_kernel_lines(asm, f"{kernel}ILi{chunks}ELi{groups}E"), chunks, table_wait)


@pytest.mark.skipif(not os.path.exists(HIPCC) or shutil.which("make") is None, reason="needs hipcc and make")
@pytest.mark.parametrize("source", ["gemv.hip", "gemv_kquant.hip", "gemm_small.hip", "quantize.hip"])
def test_kernel_arguments_preloaded(source):
    """Every kernel asks for its first kernel-argument dwords in SGPRs at wave
    launch (the build's -amdgpu-kernarg-preload-count), so a wave addresses
    memory without first waiting for a scalar load of its arguments: the c1
    GEMV takes 3.43 us with it and 3.74 us without."""
    out = os.path.join(PKG_DIR, "_build", source + ".s")
    subprocess.run(["make", "-s", "-C", PKG_DIR, out], check=True, capture_output=True, timeout=600)
    with open(out) as f:
        asm = f.read()
    lengths = [int(v) for v in re.findall(r"\.amdhsa_user_sgpr_kernarg_preload_length\s+(\d+)", asm)]
    kernels = re.findall(r"^\s*\.amdhsa_kernel\s+(\S+)", asm, re.M)
    assert kernels and len(lengths) == len(kernels), f"{len(lengths)} preload entries for {len(kernels)} kernels"
    assert all(v > 0 for v in lengths), f"kernels without preloaded arguments: {lengths.count(0)}"
