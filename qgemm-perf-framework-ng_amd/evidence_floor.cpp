// Launch and streaming-read floors of this GPU, the reference points for the
// GEMV roofline fractions: how long a kernel that does nothing takes per
// launch when replayed back to back from a graph, and how long a kernel that
// only streams N bytes from HBM (coalesced 16-byte loads, one per lane,
// rotating over enough buffer copies to defeat the 256 MB Infinity Cache)
// takes per launch. A GEMV of the same bytes cannot beat the read floor.
//
// Build: make -C qgemm-perf-framework-ng_amd pfng_floor; run ./pfng_floor.
// Prints one line per measurement and a final JSON line.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x)                                                                                   \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                                       \
        }                                                                                       \
    } while (0)

// Each lane reads one 16-byte chunk (coalesced) and folds it into a value the
// compiler cannot drop; the store never happens for real data.
__global__ __launch_bounds__(256) void stream_read(const uint4 *__restrict__ p, size_t n16, unsigned *out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const uint4 v = i < n16 ? p[i] : uint4{0, 0, 0, 0};
    if ((v.x ^ v.y ^ v.z ^ v.w) == 0x9e3779b9u) out[0] = 1;
}

__global__ void empty_kernel() {}

int main() {
    hipStream_t s;
    CK(hipStreamCreate(&s));
    unsigned *dout;
    CK(hipMalloc(&dout, 64));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));

    // empty kernel, 100 launches per graph
    double empty_us = 0;
    {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
        for (int i = 0; i < 100; ++i) hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, s);
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        CK(hipEventRecord(e0, s));
        for (int r = 0; r < 20; ++r) CK(hipGraphLaunch(ge, s));
        CK(hipEventRecord(e1, s));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        empty_us = ms * 1e3 / 2000.0;
        std::printf("empty kernel, graph replay: %.3f us per launch\n", empty_us);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }

    // streaming reads: c1's GEMV bytes, the iq2_xxs GEMV's bytes, 128 MiB
    const size_t sizes[] = {9457920, 4346432, (size_t)128 << 20};
    double read_us[3];
    for (int si = 0; si < 3; ++si) {
        const size_t bytes = sizes[si];
        const int copies = (int)(((size_t)512 << 20) / bytes) < 4 ? 4 : (int)(((size_t)512 << 20) / bytes);
        std::vector<uint4 *> bufs(copies);
        for (auto &b : bufs) {
            CK(hipMalloc(&b, bytes));
            CK(hipMemset(b, 1, bytes));
        }
        const size_t n16 = bytes / 16;
        const unsigned grid = (unsigned)((n16 + 255) / 256);
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
        for (int i = 0; i < copies; ++i)
            hipLaunchKernelGGL(stream_read, dim3(grid), dim3(256), 0, s, bufs[i], n16, dout);
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        for (int w = 0; w < 3; ++w) CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        const int reps = 2000 / copies + 1;
        CK(hipEventRecord(e0, s));
        for (int r = 0; r < reps; ++r) CK(hipGraphLaunch(ge, s));
        CK(hipEventRecord(e1, s));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        read_us[si] = ms * 1e3 / ((double)reps * copies);
        std::printf("stream read %10zu B (%d copies, %u workgroups): %.3f us per launch, %.1f GB/s\n", bytes, copies,
                    grid, read_us[si], bytes / read_us[si] / 1e3);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
        for (auto &b : bufs) CK(hipFree(b));
    }
    std::printf("{\"empty_kernel_us\": %.4f, \"read_9457920_us\": %.4f, \"read_4346432_us\": %.4f, "
                "\"read_134217728_us\": %.4f, \"read_134217728_gbs\": %.1f}\n",
                empty_us, read_us[0], read_us[1], read_us[2], ((size_t)128 << 20) / read_us[2] / 1e3);
    CK(hipFree(dout));
    return 0;
}
