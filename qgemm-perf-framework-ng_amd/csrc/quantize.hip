// Activation quantizers for gfx950: q8_0 and q8_K, byte-identical to the
// reference's llama_reference::quantize_row_q8_0 / quantize_row_q8_K
// (bench/llama_reference/llama_reference.cpp:38-52, 54-70).
//
// Both kernels are HBM-bound streaming passes (4 B read per element, 1.06 /
// 1.14 B written). Loads are 16 B per lane and consecutive lanes read
// consecutive addresses; the output is assembled in LDS so the 34- and
// 292-byte blocks leave the workgroup as contiguous dword stores. Where the
// output is 4-byte aligned those stores are written through L2 to memory
// (system-scope stores): the kernel's end then finds no dirty lines to write
// back before the product that reads them starts. Quantize + product,
// graph replays: c0 10.37 -> 10.16 us, c2 10.19 -> 9.98, c3 31.0 -> 30.5,
// M = 16 decode q4_0 7.47 -> 7.14 and iq2_xxs 7.51 -> 7.33, c4 unchanged.
// (Writing through only the q8_K quants while the bsums stayed ordinary
// 16-bit stores into the same lines cost 2-5 us instead.)
//
// Bit-exactness relies on: fmaxf for the running |x| maximum (NaNs are ignored,
// as std::max(amax, NaN) keeps amax); a correctly rounded fp32 division for
// amax / 127 and 1 / d (hipcc's default); no contraction of x * id; roundf
// (half away from zero, std::round); the ggml fp32 -> fp16 routine for d.
#include "device_common.h"
#include "kernels.h"

namespace pfng {

namespace {

constexpr int kQ8_0BlocksPerGroup = 32;  // 256 threads, 8 lanes per block
constexpr int kQ8_0GroupBytes = kQ8_0BlocksPerGroup * 34;

template <bool kAligned4>
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                           int64_t nblocks) {
    __shared__ uint16_t stage[kQ8_0GroupBytes / 2];
    const int tid = threadIdx.x;
    const int local_block = tid >> 3;
    const int sub = tid & 7;
    const int64_t block = (int64_t)blockIdx.x * kQ8_0BlocksPerGroup + local_block;
    const bool valid = block < nblocks;

    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v = *reinterpret_cast<const float4 *>(x + block * 32 + sub * 4);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = group_max<8>(amax);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint32_t q = q8_quantize4(v, id);

    // block layout in LDS: short 0 = d, shorts 1..16 = qs
    uint16_t *blk = stage + local_block * 17;
    blk[1 + sub * 2] = (uint16_t)(q & 0xffff);
    blk[2 + sub * 2] = (uint16_t)(q >> 16);
    if (sub == 0) blk[0] = (uint16_t)f32_to_fp16_bits(d);
    __syncthreads();

    const int64_t first = (int64_t)blockIdx.x * kQ8_0BlocksPerGroup;
    const int64_t nvalid = nblocks - first < kQ8_0BlocksPerGroup ? nblocks - first : kQ8_0BlocksPerGroup;
    const int bytes = (int)nvalid * 34;
    uint8_t *out = y + first * 34;
    if (kAligned4) {
        // 1088 B per full group; the group base is a multiple of 1088 (4-aligned).
        const uint32_t *src = reinterpret_cast<const uint32_t *>(stage);
        uint32_t *dst = reinterpret_cast<uint32_t *>(out);
        const int words = bytes >> 2;
        for (int i = tid; i < words; i += 256) store_through(&dst[i], src[i]);
        if ((bytes & 3) && tid == 0) reinterpret_cast<uint16_t *>(out)[bytes / 2 - 1] = stage[bytes / 2 - 1];
    } else {
        uint16_t *dst = reinterpret_cast<uint16_t *>(out);
        for (int i = tid; i < bytes / 2; i += 256) dst[i] = stage[i];
    }
}

// One wavefront per 256-element super-block; lane l owns elements 4l..4l+3.
// kAligned4: the workgroup's four blocks (1168 B, 292 dwords) are assembled
// in LDS and written as dwords through L2; otherwise each lane stores its
// parts directly.
template <bool kAligned4>
__global__ __launch_bounds__(256) void quantize_q8_K_kernel(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                           int64_t nblocks) {
    __shared__ __align__(16) uint32_t stage[4 * 292 / 4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t block = (int64_t)blockIdx.x * 4 + wave;
    if constexpr (!kAligned4) {
        if (block >= nblocks) return;
        const float4 v = *reinterpret_cast<const float4 *>(x + block * 256 + lane * 4);
        q8_K_store_lane(y + block * 292, q8_K_quantize_lane(v), lane);
    } else {
        if (block < nblocks) {
            const float4 v = *reinterpret_cast<const float4 *>(x + block * 256 + lane * 4);
            q8_K_store_lane(reinterpret_cast<uint8_t *>(stage) + wave * 292, q8_K_quantize_lane(v), lane);
        }
        __syncthreads();
        const int64_t first = (int64_t)blockIdx.x * 4;
        const int nvalid = nblocks - first < 4 ? (int)(nblocks - first) : 4;
        uint32_t *dst = reinterpret_cast<uint32_t *>(y + first * 292);
        for (int i = threadIdx.x; i < nvalid * 73; i += 256) store_through(&dst[i], stage[i]);
    }
}

}  // namespace

hipError_t launch_quantize_q8_0(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream) {
    const int64_t nblocks = rows * (k / 32);
    if (nblocks == 0) return hipSuccess;
    const int64_t groups = (nblocks + kQ8_0BlocksPerGroup - 1) / kQ8_0BlocksPerGroup;
    const bool aligned4 = (reinterpret_cast<uintptr_t>(y) & 3) == 0;
    if (aligned4)
        hipLaunchKernelGGL(quantize_q8_0_kernel<true>, dim3((unsigned)groups), dim3(256), 0, stream, x,
                           static_cast<uint8_t *>(y), nblocks);
    else
        hipLaunchKernelGGL(quantize_q8_0_kernel<false>, dim3((unsigned)groups), dim3(256), 0, stream, x,
                           static_cast<uint8_t *>(y), nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_K(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream) {
    const int64_t nblocks = rows * (k / 256);
    if (nblocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((nblocks + 3) / 4));
    if ((reinterpret_cast<uintptr_t>(y) & 3) == 0)
        hipLaunchKernelGGL(quantize_q8_K_kernel<true>, grid, dim3(256), 0, stream, x, static_cast<uint8_t *>(y), nblocks);
    else
        hipLaunchKernelGGL(quantize_q8_K_kernel<false>, grid, dim3(256), 0, stream, x, static_cast<uint8_t *>(y),
                           nblocks);
    return hipGetLastError();
}

}  // namespace pfng
