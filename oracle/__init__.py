"""TEST INFRASTRUCTURE — Python binding of the CPU oracle.

Loads oracle/build/libpfng_oracle.so (the C restatement of the reference's
scalar path, oracle/pfng_oracle.c) and, when it has been built,
oracle/_ref/libpfng_ref.so (the reference's own llama_reference.cpp and
benchmark.cpp). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module; it is the checker, never the product.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libpfng_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libpfng_ref.so")

Q4_0, Q4_K, IQ2_XXS = 0, 1, 2
TYPE_NAMES = {Q4_0: "q4_0", Q4_K: "q4_K", IQ2_XXS: "iq2_xxs"}

# Block layouts (include/pfng_blocks.h; reference include/ggml.h:125-159).
DT_Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", 16)])
DT_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
DT_Q8_K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
DT_IQ2_XXS = np.dtype([("d", "<u2"), ("qs", "<u2", 32)])
DT_Q4_K = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qs", "u1", 128)])
assert (DT_Q4_0.itemsize, DT_Q8_0.itemsize, DT_Q8_K.itemsize, DT_IQ2_XXS.itemsize, DT_Q4_K.itemsize) == (
    18, 34, 292, 66, 144)

WEIGHT_DTYPE = {Q4_0: DT_Q4_0, Q4_K: DT_Q4_K, IQ2_XXS: DT_IQ2_XXS}
ACT_DTYPE = {Q4_0: DT_Q8_0, Q4_K: DT_Q8_K, IQ2_XXS: DT_Q8_K}
QK = {Q4_0: 32, Q4_K: 256, IQ2_XXS: 256}

_c_float_p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def build(ref: bool = True) -> None:
    """Compile the oracle (and the reference wrapper when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if ref and os.path.isdir(os.environ.get("PFNG_REFERENCE", "/root/reference")):
        subprocess.run(["make", "-s", "-C", HERE, "ref",
                        "REF=" + os.environ.get("PFNG_REFERENCE", "/root/reference")], check=True)


_lib = None
_ref = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = ctypes.CDLL(LIB_PATH)
        L.pfo_fp16_to_fp32.restype = ctypes.c_float
        L.pfo_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.pfo_fp32_to_fp16.restype = ctypes.c_uint16
        L.pfo_fp32_to_fp16.argtypes = [ctypes.c_float]
        for name in ("pfo_fp16_to_fp32_n", "pfo_fp32_to_fp16_n"):
            getattr(L, name).argtypes = [_vp, _vp, _sz]
        L.pfo_mt_draws.argtypes = [ctypes.c_uint32, _vp, _sz]
        L.pfo_uniform_real_draws.argtypes = [ctypes.c_uint32, ctypes.c_float, ctypes.c_float, _vp, _sz]
        for name in ("pfo_quantize_row_q4_0", "pfo_quantize_row_q8_0", "pfo_quantize_row_q8_K",
                     "pfo_quantize_row_q4_K"):
            getattr(L, name).argtypes = [_vp, _vp, _sz]
        for name in ("pfo_quantize_q8_0", "pfo_quantize_q8_K"):
            getattr(L, name).argtypes = [_vp, _vp, _sz, _sz]
        L.pfo_dot_q4_0_q8_0.restype = ctypes.c_float
        L.pfo_dot_q4_0_q8_0.argtypes = [_vp, _vp, _sz]
        L.pfo_dot_q4_K_q8_K.restype = ctypes.c_float
        L.pfo_dot_q4_K_q8_K.argtypes = [_vp, _vp]
        L.pfo_dot_iq2_xxs_q8_K.restype = ctypes.c_float
        L.pfo_dot_iq2_xxs_q8_K.argtypes = [_vp, _vp]
        L.pfo_iq2_xxs_decode_subblock.argtypes = [_vp, _vp, ctypes.POINTER(ctypes.c_int)]
        L.pfo_q4_K_scales_mins.argtypes = [_vp, _vp, _vp]
        for name in ("pfo_isums_q4_0_q8_0", "pfo_isums_q4_K_q8_K", "pfo_isums_iq2_xxs_q8_K"):
            getattr(L, name).argtypes = [_vp, _vp, _sz, _sz, _sz, _vp]
        L.pfo_compute.restype = ctypes.c_int
        L.pfo_compute.argtypes = [ctypes.c_int, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_int]
        L.pfo_matmul.restype = ctypes.c_int
        L.pfo_matmul.argtypes = [ctypes.c_int, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_int]
        L.pfo_abs_terms.restype = ctypes.c_int
        L.pfo_abs_terms.argtypes = [ctypes.c_int, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_int]
        L.pfo_create_input.restype = ctypes.c_int
        L.pfo_create_input.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint32, _sz, _sz, _sz, _vp, _vp]
        L.pfo_checksum.restype = ctypes.c_double
        L.pfo_checksum.argtypes = [_vp, _sz]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> ctypes.CDLL:
    """The reference's own scalar code (oracle/_ref), for pinning the restatement."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_PATH)
        R.ref_fp16_to_fp32.restype = ctypes.c_float
        R.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        R.ref_fp32_to_fp16.restype = ctypes.c_uint16
        R.ref_fp32_to_fp16.argtypes = [ctypes.c_float]
        for name in ("ref_quantize_row_q4_0", "ref_quantize_row_q8_0", "ref_quantize_row_q8_K",
                     "ref_quantize_row_q4_K"):
            getattr(R, name).argtypes = [_vp, _vp, _sz]
        R.ref_dot_q4_0_q8_0.restype = ctypes.c_float
        R.ref_dot_q4_0_q8_0.argtypes = [_vp, _vp, _sz]
        R.ref_dot_q4_K_q8_K.restype = ctypes.c_float
        R.ref_dot_q4_K_q8_K.argtypes = [_vp, _vp]
        R.ref_dot_iq2_xxs_q8_K.restype = ctypes.c_float
        R.ref_dot_iq2_xxs_q8_K.argtypes = [_vp, _vp]
        R.ref_create_input.restype = ctypes.c_int
        R.ref_create_input.argtypes = [ctypes.c_int, ctypes.c_uint64, _sz, _sz, _sz, _vp, _vp]
        R.ref_compute.restype = ctypes.c_int
        R.ref_compute.argtypes = [ctypes.c_int, _vp, _vp, _vp, _sz, _sz, _sz]
        R.ref_compute_threads.restype = ctypes.c_int
        R.ref_compute_threads.argtypes = [ctypes.c_int, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_int]
        _ref = R
    return _ref


# ---------------------------------------------------------------------------
# numpy-level helpers
# ---------------------------------------------------------------------------

def fp16_to_fp32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().pfo_fp16_to_fp32_n(_ptr(h), _ptr(out), h.size)
    return out


def fp32_to_fp16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().pfo_fp32_to_fp16_n(_ptr(f), _ptr(out), f.size)
    return out


def mt_draws(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().pfo_mt_draws(seed, _ptr(out), n)
    return out


def uniform_real_draws(seed: int, a: float, b: float, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().pfo_uniform_real_draws(seed, a, b, _ptr(out), n)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """x: (rows, k) float32 -> (rows, k/32) block_q8_0 (llama_reference.cpp:38-52)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    y = np.zeros((rows, k // 32), DT_Q8_0)
    lib().pfo_quantize_q8_0(_ptr(x), _ptr(y), rows, k)
    return y


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    """x: (rows, k) float32 -> (rows, k/256) block_q8_K (llama_reference.cpp:54-70)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    y = np.zeros((rows, k // 256), DT_Q8_K)
    lib().pfo_quantize_q8_K(_ptr(x), _ptr(y), rows, k)
    return y


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(x.size // 32, DT_Q4_0)
    lib().pfo_quantize_row_q4_0(_ptr(x), _ptr(y), x.size)
    return y.reshape(x.shape[:-1] + (x.shape[-1] // 32,))


def quantize_q4_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(x.size // 256, DT_Q4_K)
    lib().pfo_quantize_row_q4_K(_ptr(x), _ptr(y), x.size)
    return y.reshape(x.shape[:-1] + (x.shape[-1] // 256,))


def quantize_activation(qtype: int, x: np.ndarray) -> np.ndarray:
    return quantize_q8_0(x) if qtype == Q4_0 else quantize_q8_K(x)


def create_input(qtype: int, m: int, n: int, k: int, seed: int = 1, variant: int = 1):
    """Seeded inputs as bench/framework/benchmark.cpp:34-94 (variant 0 = reference
    generator; variant 1 = the baseline-config iq2_xxs generator, grid 0..255, d~U[0.001,0.01))."""
    act = np.empty((m, k), np.float32)
    w = np.zeros((n, k // QK[qtype]), WEIGHT_DTYPE[qtype])
    rc = lib().pfo_create_input(qtype, variant, seed, m, n, k, _ptr(act), _ptr(w))
    if rc != 0:
        raise ValueError(f"pfo_create_input failed rc={rc}")
    return act, w


def matmul(qtype: int, w: np.ndarray, aq: np.ndarray, m: int, n: int, k: int, threads: int = 0) -> np.ndarray:
    out = np.zeros((m, n), np.float32)
    rc = lib().pfo_matmul(qtype, _ptr(w), _ptr(aq), _ptr(out), m, n, k, threads)
    if rc != 0:
        raise ValueError(f"pfo_matmul failed rc={rc}")
    return out


def compute(qtype: int, act: np.ndarray, w: np.ndarray, threads: int = 0) -> np.ndarray:
    m, k = act.shape
    n = w.shape[0]
    out = np.zeros((m, n), np.float32)
    rc = lib().pfo_compute(qtype, _ptr(np.ascontiguousarray(act)), _ptr(w), _ptr(out), m, n, k, threads)
    if rc != 0:
        raise ValueError(f"pfo_compute failed rc={rc}")
    return out


def abs_terms(qtype: int, w: np.ndarray, aq: np.ndarray, m: int, n: int, k: int, threads: int = 0) -> np.ndarray:
    out = np.zeros((m, n), np.float64)
    rc = lib().pfo_abs_terms(qtype, _ptr(w), _ptr(aq), _ptr(out), m, n, k, threads)
    if rc != 0:
        raise ValueError(f"pfo_abs_terms failed rc={rc}")
    return out


def isums(qtype: int, w: np.ndarray, aq: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    """Exact integer part of every block dot (see pfng_oracle.h)."""
    if qtype == Q4_0:
        out = np.zeros((m, n, k // 32), np.int32)
        lib().pfo_isums_q4_0_q8_0(_ptr(w), _ptr(aq), m, n, k, _ptr(out))
    elif qtype == Q4_K:
        out = np.zeros((m, n, k // 256, 2), np.int32)
        lib().pfo_isums_q4_K_q8_K(_ptr(w), _ptr(aq), m, n, k, _ptr(out))
    else:
        out = np.zeros((m, n, k // 256), np.int32)
        lib().pfo_isums_iq2_xxs_q8_K(_ptr(w), _ptr(aq), m, n, k, _ptr(out))
    return out


def checksum(out: np.ndarray) -> float:
    out = np.ascontiguousarray(out, dtype=np.float32)
    return float(lib().pfo_checksum(_ptr(out), out.size))


def within_tolerance(actual: np.ndarray, expected: np.ndarray, terms: np.ndarray, rel: float = 1e-5):
    """The fp32 output contract: |actual - expected| <= rel * sum|terms| per element.
    Returns (ok, worst_ratio, index_of_worst)."""
    err = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
    bound = rel * terms
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bound > 0, err / np.where(bound > 0, bound, 1.0), np.where(err > 0, np.inf, 0.0))
    worst = int(np.argmax(ratio)) if ratio.size else 0
    return bool(np.all(err <= bound)), float(ratio.flat[worst]) if ratio.size else 0.0, worst
