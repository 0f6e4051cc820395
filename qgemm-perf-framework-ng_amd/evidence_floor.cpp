// Launch and streaming-read floors of this GPU, the reference points for the
// GEMV roofline fractions: how long a kernel that does nothing takes per
// launch when replayed back to back from a graph, how long a kernel that only
// streams N bytes from HBM (coalesced 16-byte loads, one per lane, rotating
// over enough buffer copies to defeat the 256 MB Infinity Cache) takes per
// launch, and how long the same read takes in the M = 1 GEMV's shape (a row
// per wave) when each row also stores its result. A GEMV of the same bytes
// cannot beat the read floor, nor, with its stores, the last figure.
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

// The c1 GEMV's read shape with its store: each wave reads one 2304-byte row
// (coalesced 16-byte loads, 2.25 per lane), workgroups of 16 rows, and lane 0
// stores one float per row. Against stream_read this isolates what a kernel
// pays for writing its result at the end: the stores' completion is part of
// every GEMV's tail.
__global__ __launch_bounds__(1024) void rows_read_store(const uint8_t *__restrict__ w, float *out, int rows) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 16 + (threadIdx.x >> 6);
    const uint4 *src = reinterpret_cast<const uint4 *>(w + (size_t)row * 2304);
    const uint4 a = src[lane], b = src[lane + 64];
    const uint4 c = lane < 16 ? src[lane + 128] : uint4{0, 0, 0, 0};
    const unsigned u = a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w;
    if (lane == 0 && row < rows) out[row] = (float)(u & 0xffu);
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
    // c1's weight matrix (4096 rows of 2304 bytes) read row per wave, one float stored per row
    double rows_store_us = 0;
    {
        const int rows = 4096;
        const size_t bytes = (size_t)rows * 2304;
        const int copies = 32;
        std::vector<uint8_t *> bufs(copies);
        for (auto &b : bufs) {
            CK(hipMalloc(&b, bytes));
            CK(hipMemset(b, 1, bytes));
        }
        float *out;
        CK(hipMalloc(&out, rows * sizeof(float)));
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
        for (int i = 0; i < copies; ++i)
            hipLaunchKernelGGL(rows_read_store, dim3(rows / 16), dim3(1024), 0, s, bufs[i], out, rows);
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        for (int w = 0; w < 3; ++w) CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        const int reps = 100;
        CK(hipEventRecord(e0, s));
        for (int r = 0; r < reps; ++r) CK(hipGraphLaunch(ge, s));
        CK(hipEventRecord(e1, s));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        rows_store_us = ms * 1e3 / ((double)reps * copies);
        std::printf("row-per-wave read of %zu B + one float stored per row (%d copies, %d workgroups): %.3f us per launch\n",
                    bytes, copies, rows / 16, rows_store_us);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
        for (auto &b : bufs) CK(hipFree(b));
        CK(hipFree(out));
    }
    std::printf("{\"empty_kernel_us\": %.4f, \"read_9457920_us\": %.4f, \"read_4346432_us\": %.4f, "
                "\"read_134217728_us\": %.4f, \"read_134217728_gbs\": %.1f, \"rows_read_store_9437184_us\": %.4f}\n",
                empty_us, read_us[0], read_us[1], read_us[2], ((size_t)128 << 20) / read_us[2] / 1e3, rows_store_us);
    CK(hipFree(dout));
    return 0;
}
