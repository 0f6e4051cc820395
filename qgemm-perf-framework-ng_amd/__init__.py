"""qgemm-perf-framework-ng_amd — MI355X (gfx950) backend for the quantized GGML GEMM path.

Python binding of the C-ABI in include/pfng_hip.h (libpfng_hip.so, built
in-tree by the Makefile beside this file). The library operates on device
memory; this module passes torch tensors' device pointers and the current HIP
stream. Block buffers are uint8 tensors holding the GGML block bytes
(include/pfng_blocks.h), shaped (rows, blocks_per_row * block_bytes).

There is no CPU fallback: every call goes to the HIP library, and loading
fails loudly when libpfng_hip.so is missing.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpfng_hip.so")

# pfng_quantization_type (include/pfng_blocks.h), numbered as the reference's QuantizationType
Q4_0, Q4_K, IQ2_XXS = 0, 1, 2
TYPE_NAMES = {Q4_0: "q4_0", Q4_K: "q4_K", IQ2_XXS: "iq2_xxs"}
# pfng_path
PATH_AUTO, PATH_GEMV, PATH_MFMA, PATH_NAIVE = 0, 1, 2, 3
PATH_NAMES = {PATH_AUTO: "auto", PATH_GEMV: "gemv", PATH_MFMA: "mfma", PATH_NAIVE: "naive"}
# pfng_status
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_HIP, ERR_DEVICE = 0, 1, 2, 3, 4

QK = {Q4_0: 32, Q4_K: 256, IQ2_XXS: 256}
WEIGHT_BLOCK_BYTES = {Q4_0: 18, Q4_K: 144, IQ2_XXS: 66}
ACT_BLOCK_BYTES = {Q4_0: 34, Q4_K: 292, IQ2_XXS: 292}


class PfngError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"pfng status {status}: {message}")
        self.status = status


def build(jobs: int = 8) -> None:
    """Compile libpfng_hip.so for gfx950 (hipcc cross-compiles without a GPU)."""
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}"], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` (no CPU fallback exists)")
        # torch carries its own HIP runtime (torch/lib/libamdhip64.so, soname
        # libamdhip64.so.7, which torch's libraries name without the version).
        # Loaded first, it satisfies the library's libamdhip64.so.7 and both
        # share one runtime; loaded after the library, it would come in as a
        # second runtime beside ROCm's, and the library's runtime then fails on
        # the device torch holds. The tensors and streams this binding passes
        # belong to torch's runtime, so load torch first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, sz, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_int
        L.pfng_hip_last_error.restype = ctypes.c_char_p
        L.pfng_hip_version.restype = ctypes.c_char_p
        L.pfng_hip_device_check.argtypes = [ctypes.c_char_p, sz, ctypes.POINTER(ctypes.c_int)]
        for name in ("pfng_hip_quantize_q8_0", "pfng_hip_quantize_q8_K", "pfng_hip_quantize_q4_0",
                     "pfng_hip_quantize_q4_K"):
            getattr(L, name).argtypes = [vp, vp, i64, i64, vp]
        for name in ("pfng_hip_mul_mat_q4_0_q8_0", "pfng_hip_mul_mat_q4_K_q8_K", "pfng_hip_mul_mat_iq2_xxs_q8_K"):
            getattr(L, name).argtypes = [vp, vp, vp, i64, i64, i64, ci, vp]
        L.pfng_hip_mul_mat.argtypes = [ci, vp, vp, vp, i64, i64, i64, ci, vp]
        L.pfng_hip_auto_path.argtypes = [ci, i64, i64, i64]
        L.pfng_hip_compute_workspace_size.restype = sz
        L.pfng_hip_compute_workspace_size.argtypes = [ci, i64, i64]
        L.pfng_hip_compute.argtypes = [ci, vp, vp, vp, i64, i64, i64, vp, sz, ci, vp]
        L.pfng_hip_compute_noalloc.argtypes = [ci, vp, vp, vp, i64, i64, i64, ci, vp]
        L.pfng_hip_block_isums.argtypes = [ci, vp, vp, vp, i64, i64, i64, vp]
        L.pfng_host_create_input.argtypes = [ci, ci, ctypes.c_uint32, sz, sz, sz, vp, vp]
        L.pfng_host_quantize_weights.argtypes = [ci, vp, vp, sz, sz]
        L.pfng_host_compute.argtypes = [ci, vp, vp, vp, sz, sz, sz, sz]
        L.pfng_host_fp32_to_fp16.restype = ctypes.c_uint16
        L.pfng_host_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.pfng_host_fp16_to_fp32.restype = ctypes.c_float
        L.pfng_host_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.pfng_host_checksum.restype = ctypes.c_double
        L.pfng_host_checksum.argtypes = [vp, sz]
        _lib = L
    return _lib


# C-ABI symbols declared in include/pfng_hip.h
EXPORTED_SYMBOLS = (
    "pfng_hip_last_error", "pfng_hip_version", "pfng_hip_device_check",
    "pfng_hip_quantize_q8_0", "pfng_hip_quantize_q8_K", "pfng_hip_quantize_q4_0", "pfng_hip_quantize_q4_K",
    "pfng_hip_mul_mat_q4_0_q8_0", "pfng_hip_mul_mat_q4_K_q8_K", "pfng_hip_mul_mat_iq2_xxs_q8_K",
    "pfng_hip_mul_mat", "pfng_hip_auto_path", "pfng_hip_compute_workspace_size", "pfng_hip_compute",
    "pfng_hip_compute_noalloc", "pfng_hip_block_isums",
)
# host-side C-ABI declared in include/pfng_host.h
HOST_SYMBOLS = (
    "pfng_host_create_input", "pfng_host_quantize_weights", "pfng_host_compute", "pfng_host_fp32_to_fp16",
    "pfng_host_fp16_to_fp32", "pfng_host_checksum",
)
INPUT_REFERENCE, INPUT_BASELINE = 0, 1


def last_error() -> str:
    return lib().pfng_hip_last_error().decode()


def check(status: int) -> None:
    if status != OK:
        raise PfngError(status, last_error())


def version() -> str:
    return lib().pfng_hip_version().decode()


def device_check() -> tuple[str, int]:
    arch = ctypes.create_string_buffer(64)
    cus = ctypes.c_int(0)
    check(lib().pfng_hip_device_check(arch, 64, ctypes.byref(cus)))
    return arch.value.decode(), cus.value


# ---------------------------------------------------------------------------
# host-side input generation (bench/framework/benchmark.cpp:29-94)
# ---------------------------------------------------------------------------

def create_input(qtype: int, m: int, n: int, k: int, seed: int = 1, variant: int = INPUT_BASELINE):
    """Synthetic inputs as the reference harness makes them: returns (activation
    float32 (m, k), weight uint8 (n, k/QK * block_bytes)) as numpy arrays."""
    import numpy as np
    act = np.empty((m, k), np.float32)
    w = np.empty((n, (k // QK[qtype]) * WEIGHT_BLOCK_BYTES[qtype]), np.uint8)
    rc = lib().pfng_host_create_input(qtype, variant, seed, m, n, k, act.ctypes.data, w.ctypes.data)
    if rc != 0:
        raise ValueError(f"pfng_host_create_input({TYPE_NAMES.get(qtype, qtype)}, m={m}, n={n}, k={k}) failed: {rc}")
    return act, w


def quantize_weights(qtype: int, x):
    """Host weight quantizer of the reference (q4_0 or q4_K): float32 (rows, k)
    -> uint8 (rows, k/QK * block_bytes)."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    y = np.empty((rows, (k // QK[qtype]) * WEIGHT_BLOCK_BYTES[qtype]), np.uint8)
    rc = lib().pfng_host_quantize_weights(qtype, x.ctypes.data, y.ctypes.data, rows, k)
    if rc != 0:
        raise ValueError(f"pfng_host_quantize_weights({TYPE_NAMES.get(qtype, qtype)}, k={k}) failed: {rc}")
    return y


def host_compute(qtype: int, activation, weight, n: int, threads: int = 1):
    """llama_reference::compute on the host (the harness's verification
    reference): float32 (m, k) activations and uint8 weight blocks -> float32 (m, n)."""
    import numpy as np
    act = np.ascontiguousarray(activation, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.uint8)
    m, k = act.shape
    out = np.empty((m, n), np.float32)
    if qtype in QK and k % QK[qtype] == 0 and w.nbytes < n * (k // QK[qtype]) * WEIGHT_BLOCK_BYTES[qtype]:
        raise ValueError("weight buffer is smaller than n rows of k/QK blocks")
    rc = lib().pfng_host_compute(qtype, act.ctypes.data, w.ctypes.data, out.ctypes.data, m, n, k, threads)
    if rc != 0:
        raise ValueError(f"pfng_host_compute({TYPE_NAMES.get(qtype, qtype)}, m={m}, n={n}, k={k}) failed: {rc}")
    return out


def checksum(out) -> float:
    """Sum of every 257th output (kernels/common/adapter_common.cpp:18-23)."""
    import numpy as np
    out = np.ascontiguousarray(out, dtype=np.float32)
    return float(lib().pfng_host_checksum(out.ctypes.data, out.size))


# ---------------------------------------------------------------------------
# torch-level helpers (torch is plumbing: device memory and streams)
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _stream(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _p(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _need(t, nbytes: int, name: str) -> None:
    """The C-ABI takes bare device pointers: check here that a tensor is a
    contiguous device tensor holding at least `nbytes` bytes."""
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    have = t.numel() * t.element_size()
    if have < nbytes:
        raise ValueError(f"{name} holds {have} bytes, {nbytes} needed")


def _blocks(qtype: int, rows: int, k: int, weight: bool) -> int:
    per = WEIGHT_BLOCK_BYTES[qtype] if weight else ACT_BLOCK_BYTES[qtype]
    return rows * (k // QK[qtype]) * per


def quantize_q8_0(x, out=None, stream=None):
    """x: (rows, k) float32 CUDA tensor -> (rows, k/32*34) uint8 block_q8_0 bytes."""
    torch = _torch()
    rows, k = x.shape
    if out is None:
        out = torch.empty((rows, (k // 32) * 34), dtype=torch.uint8, device=x.device)
    _need(x, rows * k * 4, "x")
    _need(out, _blocks(Q4_0, rows, k, False), "out")
    check(lib().pfng_hip_quantize_q8_0(_p(x), _p(out), rows, k, _stream(stream)))
    return out


def quantize_weights_gpu(qtype: int, x, out=None, stream=None):
    """Reference weight quantizer on the device: x (rows, k) float32 CUDA tensor
    -> (rows, k/QK * block_bytes) uint8 block bytes (q4_0 or q4_K)."""
    torch = _torch()
    rows, k = x.shape
    if out is None:
        out = torch.empty((rows, (k // QK[qtype]) * WEIGHT_BLOCK_BYTES[qtype]), dtype=torch.uint8, device=x.device)
    fn = {Q4_0: lib().pfng_hip_quantize_q4_0, Q4_K: lib().pfng_hip_quantize_q4_K}[qtype]
    _need(x, rows * k * 4, "x")
    _need(out, _blocks(qtype, rows, k, True), "out")
    check(fn(_p(x), _p(out), rows, k, _stream(stream)))
    return out


def quantize_q8_K(x, out=None, stream=None):
    """x: (rows, k) float32 CUDA tensor -> (rows, k/256*292) uint8 block_q8_K bytes."""
    torch = _torch()
    rows, k = x.shape
    if out is None:
        out = torch.empty((rows, (k // 256) * 292), dtype=torch.uint8, device=x.device)
    _need(x, rows * k * 4, "x")
    _need(out, _blocks(Q4_K, rows, k, False), "out")
    check(lib().pfng_hip_quantize_q8_K(_p(x), _p(out), rows, k, _stream(stream)))
    return out


def quantize_activation(qtype: int, x, out=None, stream=None):
    return quantize_q8_0(x, out, stream) if qtype == Q4_0 else quantize_q8_K(x, out, stream)


def mul_mat(qtype: int, weight, act_q, m: int, n: int, k: int, path: int = PATH_AUTO, out=None, stream=None):
    """C (m, n) float32 = W (n x k, quantized) . A (m x k, q8)^T on the GPU."""
    torch = _torch()
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=weight.device)
    if qtype in QK and m > 0 and n > 0 and k > 0 and k % QK[qtype] == 0:  # other shapes: the library reports the error
        _need(weight, _blocks(qtype, n, k, True), "weight")
        _need(act_q, _blocks(qtype, m, k, False), "act_q")
        _need(out, m * n * 4, "out")
    check(lib().pfng_hip_mul_mat(qtype, _p(weight), _p(act_q), _p(out), m, n, k, path, _stream(stream)))
    return out


def auto_path(qtype: int, m: int, n: int, k: int) -> int:
    """The path PATH_AUTO takes for this shape (aligned operands): PATH_GEMV or
    PATH_MFMA, PATH_AUTO for an empty product, or -1 when PATH_AUTO declines it
    (only PATH_NAIVE runs such a shape). Touches no device."""
    return lib().pfng_hip_auto_path(qtype, m, n, k)


def compute(qtype: int, activation, weight, n: int, path: int = PATH_AUTO, out=None, workspace=None, stream=None):
    """llama_reference::compute on the GPU: quantize fp32 activations, then the product."""
    torch = _torch()
    m, k = activation.shape
    need = lib().pfng_hip_compute_workspace_size(qtype, m, k)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=activation.device)
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=activation.device)
    if qtype in QK and m > 0 and n > 0 and k > 0 and k % QK[qtype] == 0:
        _need(activation, m * k * 4, "activation")
        _need(weight, _blocks(qtype, n, k, True), "weight")
        _need(out, m * n * 4, "out")
        _need(workspace, need, "workspace")
    check(lib().pfng_hip_compute(qtype, _p(activation), _p(weight), _p(out), m, n, k, _p(workspace),
                                 workspace.numel(), path, _stream(stream)))
    return out


def compute_noalloc(qtype: int, activation, weight, n: int, path: int = PATH_AUTO, out=None, stream=None):
    """compute() without a workspace: the library's static per-device scratch
    holds the quantized activations (at most 16 MiB of them)."""
    torch = _torch()
    m, k = activation.shape
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=activation.device)
    if qtype in QK and m > 0 and n > 0 and k > 0 and k % QK[qtype] == 0:
        _need(activation, m * k * 4, "activation")
        _need(weight, _blocks(qtype, n, k, True), "weight")
        _need(out, m * n * 4, "out")
    check(lib().pfng_hip_compute_noalloc(qtype, _p(activation), _p(weight), _p(out), m, n, k, path, _stream(stream)))
    return out


def block_isums(qtype: int, weight, act_q, m: int, n: int, k: int, stream=None):
    """Exact integer parts of every block dot (diagnostic; see include/pfng_hip.h)."""
    torch = _torch()
    nb = k // QK[qtype]
    shape = (m, n, nb, 2) if qtype == Q4_K else (m, n, nb)
    out = torch.empty(shape, dtype=torch.int32, device=weight.device)
    if qtype in QK and m > 0 and n > 0 and k > 0 and k % QK[qtype] == 0:
        _need(weight, _blocks(qtype, n, k, True), "weight")
        _need(act_q, _blocks(qtype, m, k, False), "act_q")
    check(lib().pfng_hip_block_isums(qtype, _p(weight), _p(act_q), _p(out), m, n, k, _stream(stream)))
    return out
