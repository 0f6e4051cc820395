"""pfng_hip_compute_noalloc: pfng_hip_compute without a workspace, for callers
that cannot allocate. Its quantized activations live in the library's static
per-device scratch array; the results must equal pfng_hip_compute's (same
kernels, same inputs: bit for bit), call after call, also when a call follows a
larger one whose bytes are still in the scratch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

SCRATCH_BYTES = 16 << 20


def test_noalloc_rejects_shapes_beyond_the_scratch(pkg):
    """No device work: the size check comes first."""
    L = pkg.lib()
    fake = ctypes.c_void_p(256)
    # q4_0: m * (k/32) * 34 bytes; 4096 rows of k = 4096 need 17.0 MiB
    assert L.pfng_hip_compute_noalloc(0, fake, fake, fake, 4096, 8, 4096, 0, None) == pkg.ERR_INVALID_ARGUMENT
    assert "16777216-byte static scratch" in pkg.last_error()
    # q8_K: m * (k/256) * 292 bytes
    assert L.pfng_hip_compute_noalloc(1, fake, fake, fake, 4096, 8, 4096, 0, None) == pkg.ERR_INVALID_ARGUMENT
    assert L.pfng_hip_compute_noalloc(0, fake, fake, fake, 4, 8, 48, 0, None) == pkg.ERR_INVALID_ARGUMENT
    assert L.pfng_hip_compute_noalloc(0, fake, fake, fake, 0, 8, 64, 0, None) == pkg.OK
    # the boundary at k = 4096: 3855 rows take 16,776,960 bytes, 3856 rows 16,781,312
    assert L.pfng_hip_compute_workspace_size(0, 3855, 4096) <= SCRATCH_BYTES < L.pfng_hip_compute_workspace_size(0, 3856, 4096)
    assert L.pfng_hip_compute_noalloc(0, fake, fake, fake, 3856, 8, 4096, 0, None) == pkg.ERR_INVALID_ARGUMENT
    assert "16781312 bytes" in pkg.last_error()
    # 3855 rows pass the size check. Null operands make a later host check end
    # the call (no device: the scratch lookup; a device: the quantizer's null
    # check), so nothing is launched on either kind of machine; fake non-null
    # pointers would reach a kernel launch on a GPU box.
    rc = L.pfng_hip_compute_noalloc(0, None, None, None, 3855, 8, 4096, 0, None)
    assert rc != pkg.OK and "static scratch" not in pkg.last_error()


# (qtype, m, n, k, variant): each type's first call fills more of the scratch
# than its second; all go through the separate quantize launch (m >= 3)
CASES = [
    (0, 96, 256, 2048, 0), (0, 8, 192, 1024, 0),
    (1, 40, 128, 2048, 0), (1, 5, 96, 1024, 0),
    (2, 33, 128, 2048, 1), (2, 9, 64, 1024, 1),
]


@pytest.mark.gpu
def test_noalloc_matches_compute(hip, torch_gpu):
    torch = torch_gpu
    for qtype, m, n, k, variant in CASES:
        print(f"[case] compute_noalloc type={qtype} {m}x{n}x{k}", flush=True)
        act, w = hip.create_input(qtype, m, n, k, seed=3 + m, variant=variant)
        a_t = torch.from_numpy(act).cuda()
        w_t = torch.from_numpy(np.ascontiguousarray(w)).cuda()
        expect = hip.compute(qtype, a_t, w_t, n)
        got = hip.compute_noalloc(qtype, a_t, w_t, n)
        again = hip.compute_noalloc(qtype, a_t, w_t, n)
        torch.cuda.synchronize()
        e = expect.cpu().numpy()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), e.view(np.uint32)), (qtype, m, n, k)
        assert np.array_equal(again.cpu().numpy().view(np.uint32), e.view(np.uint32)), (qtype, m, n, k)


@pytest.mark.gpu
def test_noalloc_largest_shape_and_naive_path(hip, torch_gpu):
    """The largest q4_0 shape the scratch takes at k = 4096 (3855 rows, all
    but 256 bytes of it), then a small call on the naive path: both equal
    pfng_hip_compute."""
    torch = torch_gpu
    for m, n, k, path in ((3855, 64, 4096, hip.PATH_AUTO), (3, 40, 512, hip.PATH_NAIVE)):
        print(f"[case] compute_noalloc q4_0 {m}x{n}x{k} path={path}", flush=True)
        act, w = hip.create_input(0, m, n, k, seed=11, variant=0)
        a_t = torch.from_numpy(act).cuda()
        w_t = torch.from_numpy(np.ascontiguousarray(w)).cuda()
        expect = hip.compute(0, a_t, w_t, n, path=path)
        got = hip.compute_noalloc(0, a_t, w_t, n, path=path)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), expect.cpu().numpy().view(np.uint32))


@pytest.mark.gpu
def test_noalloc_under_graph_capture(hip, torch_gpu):
    """compute_noalloc captured into a graph (the scratch address was resolved
    by pfng_hip_device_check before): every replay, with other eager work and
    synchronizations between replays, equals pfng_hip_compute bit for bit. The
    fused (m = 1) and the separate-quantize (m = 24) forms."""
    torch = torch_gpu
    for qtype, m, n, k in ((0, 1, 512, 4096), (0, 24, 256, 2048), (1, 24, 256, 2048)):
        print(f"[case] compute_noalloc graph type={qtype} {m}x{n}x{k}", flush=True)
        act, w = hip.create_input(qtype, m, n, k, seed=5, variant=0)
        a_t = torch.from_numpy(act).cuda()
        w_t = torch.from_numpy(np.ascontiguousarray(w)).cuda()
        expect = hip.compute(qtype, a_t, w_t, n)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            hip.compute_noalloc(qtype, a_t, w_t, n, out=out)
        for _ in range(3):
            out.zero_()
            hip.compute(qtype, a_t[: max(1, m // 2)].contiguous(), w_t, n)  # other work through the same kernels
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint32), expect.cpu().numpy().view(np.uint32))
