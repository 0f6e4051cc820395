"""The C-ABI library loads, exports every symbol include/*.h declares, and rejects
bad arguments before touching the device — CPU only (no kernel launches)."""
from __future__ import annotations

import ctypes
import glob
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(h).read()
        for m in re.finditer(r"^\s*(?:const\s+)?[\w\s\*]+?\b(pfng_(?:hip|host)_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_the_abi():
    names = declared_symbols()
    assert "pfng_hip_mul_mat_q4_0_q8_0" in names and "pfng_hip_quantize_q8_K" in names
    assert len(names) >= 12


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.lib()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert set(declared_symbols()) <= exported
    assert set(pkg.EXPORTED_SYMBOLS) | set(pkg.HOST_SYMBOLS) == set(declared_symbols())


def test_version_string(pkg):
    assert "gfx950" in pkg.version()


@pytest.mark.parametrize("call,expect", [
    (lambda L: L.pfng_hip_quantize_q8_0(None, None, 4, 33, None), 1),
    (lambda L: L.pfng_hip_quantize_q8_0(None, None, -1, 32, None), 1),
    (lambda L: L.pfng_hip_quantize_q8_0(None, None, 0, 32, None), 0),
    (lambda L: L.pfng_hip_quantize_q8_K(None, None, 2, 128, None), 1),
    (lambda L: L.pfng_hip_quantize_q4_0(None, None, 2, 48, None), 1),
    (lambda L: L.pfng_hip_quantize_q4_0(None, None, 0, 64, None), 0),
    (lambda L: L.pfng_hip_quantize_q4_K(ctypes.c_void_p(16), ctypes.c_void_p(8), 2, 256, None), 1),
    (lambda L: L.pfng_hip_quantize_q4_K(None, None, 1, 384, None), 1),
    (lambda L: L.pfng_hip_quantize_q8_K(ctypes.c_void_p(16), ctypes.c_void_p(3), 2, 256, None), 1),
    (lambda L: L.pfng_hip_mul_mat(7, None, None, None, 1, 1, 32, 0, None), 1),
    (lambda L: L.pfng_hip_mul_mat(0, None, None, None, 1, 1, 48, 0, None), 1),
    (lambda L: L.pfng_hip_mul_mat(1, None, None, None, 1, 1, 512 + 32, 0, None), 1),
    (lambda L: L.pfng_hip_mul_mat(0, None, None, None, 0, 5, 32, 0, None), 0),
    (lambda L: L.pfng_hip_mul_mat(0, None, None, None, 4, 4, 64, 0, None), 1),
    (lambda L: L.pfng_hip_mul_mat(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 4, 4, 64, 9, None), 1),
    (lambda L: L.pfng_hip_mul_mat(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 64, 4, 96, 2, None), 2),
    # the GEMV takes up to m = 16 (m > 8 only while the activations fit in LDS),
    # up to m = 128 at k % 4096 == 0; k = 20736 is 81 super-blocks
    (lambda L: L.pfng_hip_mul_mat(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 17, 4, 256, 1, None), 2),
    (lambda L: L.pfng_hip_mul_mat(1, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 17, 4, 256, 1, None), 2),
    (lambda L: L.pfng_hip_mul_mat(2, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 9, 4, 20736, 1, None), 2),
    (lambda L: L.pfng_hip_mul_mat(2, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 129, 4, 8192, 1, None), 2),
    # the automatic path declines what no tiled path takes instead of falling
    # back to the one-thread-per-output kernel
    (lambda L: L.pfng_hip_mul_mat(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 17, 4, 96, 0, None), 2),
    (lambda L: L.pfng_hip_mul_mat(0, ctypes.c_void_p(258), ctypes.c_void_p(256), ctypes.c_void_p(256), 1, 4, 64, 0, None), 2),
    (lambda L: L.pfng_hip_mul_mat(1, ctypes.c_void_p(256), ctypes.c_void_p(264), ctypes.c_void_p(256), 64, 4, 256, 0, None), 2),
    (lambda L: L.pfng_hip_compute(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 3, 5, 96,
                                  ctypes.c_void_p(256), 3 * 3 * 34, 0, None), 2),
    (lambda L: L.pfng_hip_compute(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 4, 4, 64, None, 10, 0, None), 1),
    (lambda L: L.pfng_hip_block_isums(0, ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), 4, 4, 96, None), 2),
])
def test_argument_validation(pkg, call, expect):
    L = pkg.lib()
    assert call(L) == expect
    if expect:
        assert pkg.last_error()


@pytest.mark.parametrize("qtype,m,n,k,expect", [
    (0, 1, 4096, 4096, 1), (0, 16, 4096, 4096, 1), (0, 17, 4096, 4096, 1), (0, 64, 4096, 4096, 1),
    (0, 128, 4096, 4096, 1), (0, 129, 4096, 4096, 2), (0, 480, 1536, 1536, 2),
    (0, 3, 5, 96, -1), (0, 17, 8, 96, -1), (0, 24, 32, 256, 2), (0, 0, 8, 64, 0),
    (1, 8, 64, 512, 1), (1, 480, 1536, 1536, 2), (2, 512, 4096, 4096, 2), (2, 1, 4096, 4096, 1),
    # the GEMV path runs MFMA tiles over chunks of 16 activation rows (one K group
    # per wave and round) up to m = 128 from k = 2048 and up to m = 64 below, for
    # q4_0 at k % 256 == 0 from 512, q4_K at k % 1024 == 0 and iq2_xxs at
    # k % 2048 == 0; other k take the GEMM from m = 17
    (1, 32, 4096, 4096, 1), (2, 128, 4096, 4096, 1), (2, 129, 4096, 4096, 2), (1, 17, 4096, 8192, 1),
    (0, 17, 4096, 8192, 1), (0, 64, 4096, 12288, 1), (2, 16, 4096, 8192, 1), (1, 12, 4096, 12288, 1),
    (1, 129, 4096, 8192, 2), (0, 17, 4096, 6144, 1), (2, 17, 4096, 6144, 1), (0, 12, 4096, 14336, 1),
    (0, 17, 4096, 4352, 1), (0, 128, 4096, 11008, 1), (0, 17, 4096, 3840, 1), (1, 17, 4096, 5120, 1),
    (0, 64, 4096, 1024, 1), (0, 65, 4096, 1024, 2), (0, 128, 4096, 2048, 1), (0, 17, 4096, 256, 2),
    (1, 64, 4096, 1024, 1), (1, 65, 4096, 1024, 2), (1, 128, 4096, 3072, 1), (2, 128, 4096, 2048, 1),
    (1, 17, 4096, 4352, 2), (2, 17, 4096, 5120, 2), (2, 64, 4096, 14336, 1), (1, 16, 4096, 14336, 1),
    (0, 4, 4, 48, -1), (3, 4, 4, 64, -1),
])
def test_auto_path_query(pkg, qtype, m, n, k, expect):
    """pfng_hip_auto_path names the path PFNG_PATH_AUTO runs, or -1 where it declines."""
    assert pkg.auto_path(qtype, m, n, k) == expect
    if expect < 0:
        assert pkg.last_error()


@pytest.mark.parametrize("qtype,m", [(0, 1), (0, 16), (0, 100), (0, 480), (1, 1), (1, 40), (1, 480), (2, 8), (2, 512)])
def test_tiled_paths_stop_at_the_32_bit_offset_limit(pkg, qtype, m):
    """The tiled kernels address a tile's rows with 32-bit byte offsets, valid
    up to k = 2^24: the automatic path takes k = 2^24 and declines the next
    valid k (only the naive path runs it), naming the limit."""
    limit = 1 << 24
    assert pkg.auto_path(qtype, m, 64, limit) in (1, 2)
    assert pkg.auto_path(qtype, m, 64, limit + 256) == -1
    assert "k <= 16777216" in pkg.last_error()
    L = pkg.lib()
    p = ctypes.c_void_p(256)
    for path in (1, 2):
        assert L.pfng_hip_mul_mat(qtype, p, p, p, m, 64, limit + 256, path, None) == pkg.ERR_UNSUPPORTED
        assert "k <= 16777216" in pkg.last_error()


@pytest.mark.parametrize("qtype,m,k,path,text", [
    (0, 17, 96, 0, "m = 9..64 (k < 2048) or 9..128 at k%256==0 from k = 512"),
    (0, 129, 4096, 1, "the q4_0 GEMV takes m == 1 at k%64==0"),
    (1, 129, 8192, 1, "m = 9..64 at k = 1024 and 9..128 at k%1024==0"),
    (2, 17, 5120, 1, "m = 9..128 at k%2048==0"),
    (0, 17, 96, 2, "the q4_0 MFMA GEMM takes k%128==0"),
])
def test_declined_shapes_name_the_rules(pkg, qtype, m, k, path, text):
    """A declined shape's message states the shapes the paths do take (the GEMV
    runs up to m = 128 at the tiles' k, not only m <= 16)."""
    p = ctypes.c_void_p(256)
    assert pkg.lib().pfng_hip_mul_mat(qtype, p, p, p, m, 64, k, path, None) == pkg.ERR_UNSUPPORTED
    assert text in pkg.last_error(), pkg.last_error()
    assert "m<=16" not in pkg.last_error()


def test_workspace_size(pkg):
    L = pkg.lib()
    assert L.pfng_hip_compute_workspace_size(0, 3, 64) == 3 * 2 * 34
    assert L.pfng_hip_compute_workspace_size(1, 3, 512) == 3 * 2 * 292
    assert L.pfng_hip_compute_workspace_size(2, 0, 512) == 0


def test_auto_path_sweep(pkg):
    """The automatic path over a grid of shapes follows the documented rules:
    every shape with m <= 8 and k % 256 == 0 takes the GEMV; the MFMA tile
    GEMVs take m up to 64 below k = 2048 and 128 from there, at q4_0 k % 256
    (from 512), q4_K k % 1024 and iq2_xxs k % 2048; past those m the GEMM takes
    over (q4_0 needs k % 128 there, which k % 256 gives)."""
    for qtype in (0, 1, 2):
        unit = {0: 256, 1: 1024, 2: 2048}[qtype]
        for k in (256, 512, 768, 1024, 1536, 2048, 3072, 4096, 4352, 5120, 6144, 8192, 11008, 14336, 16384):
            tiles = k % unit == 0 and k >= (512 if qtype == 0 else unit)
            max_m = 128 if k >= 2048 else 64
            for m in list(range(1, 18)) + [31, 32, 33, 63, 64, 65, 96, 127, 128, 129, 160]:
                got = pkg.auto_path(qtype, m, 4096, k)
                assert got in (1, 2), (qtype, m, k, got)
                if m <= 8:
                    assert got == 1, (qtype, m, k)
                if 9 <= m <= max_m and tiles:
                    assert got == 1, (qtype, m, k)
                if m > 16 and not (tiles and m <= max_m):
                    assert got == 2, (qtype, m, k)
