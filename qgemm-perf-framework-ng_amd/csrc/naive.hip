// One thread per output element, evaluating the reference's scalar dot
// products (bench/llama_reference/llama_reference.cpp:113-161) with the same
// fp32 operation order and no contraction, so its output is bit-identical to
// llama_reference::compute for the same quantized operands. It is the fallback
// for shapes the tiled paths do not take and a device-side cross-check.
#include "device_common.h"
#include "kernels.h"
#include "pfng_iq2xxs_grid.h"

#pragma clang fp contract(off)

namespace pfng {

namespace {

// llama_reference.cpp:134-146
__global__ void naive_q4_0_kernel(const pfng_block_q4_0 *__restrict__ w, const pfng_block_q8_0 *__restrict__ a,
                                  float *__restrict__ c, int64_t m, int64_t n, int64_t nb) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    const int64_t mi = idx / n, ni = idx % n;
    const pfng_block_q4_0 *wr = w + ni * nb;
    const pfng_block_q8_0 *ar = a + mi * nb;
    float sum = 0.0f;
    for (int64_t b = 0; b < nb; ++b) {
        int32_t isum = 0;
        for (int i = 0; i < 16; ++i) {
            const int q = wr[b].qs[i];
            isum += ((q & 15) - 8) * ar[b].qs[i];
            isum += ((q >> 4) - 8) * ar[b].qs[i + 16];
        }
        const float t0 = mul_rn((float)isum, fp16_to_f32(wr[b].d));
        const float t1 = mul_rn(t0, fp16_to_f32(ar[b].d));
        sum = add_rn(sum, t1);
    }
    c[idx] = sum;
}

// llama_reference.cpp:113-132, accumulated over super-blocks as :186-189
__global__ void naive_q4_K_kernel(const pfng_block_q4_K *__restrict__ w, const pfng_block_q8_K *__restrict__ a,
                                  float *__restrict__ c, int64_t m, int64_t n, int64_t nb) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    const int64_t mi = idx / n, ni = idx % n;
    float out = 0.0f;
    for (int64_t b = 0; b < nb; ++b) {
        const pfng_block_q4_K &wb = w[ni * nb + b];
        const pfng_block_q8_K &ab = a[mi * nb + b];
        uint8_t scales[8], mins[8];
        for (int i = 0; i < 4; ++i) {
            scales[i] = wb.scales[i] & 63;
            scales[i + 4] = (uint8_t)((wb.scales[i + 8] & 15) | ((wb.scales[i] >> 6) << 4));
            mins[i] = wb.scales[i + 4] & 63;
            mins[i + 4] = (uint8_t)((wb.scales[i + 8] >> 4) | ((wb.scales[i + 4] >> 6) << 4));
        }
        const float d = fp16_to_f32(wb.d), dmin = fp16_to_f32(wb.dmin);
        float sum = 0.0f;
        for (int sb = 0; sb < 8; ++sb)
            for (int j = 0; j < 32; ++j) {
                const uint8_t packed = wb.qs[(sb / 2) * 32 + j];
                const int q = (sb % 2 == 0) ? (packed & 15) : (packed >> 4);
                const float t0 = mul_rn(d, (float)scales[sb]);
                const float t1 = mul_rn(t0, (float)q);
                const float t2 = mul_rn(dmin, (float)mins[sb]);
                const float t3 = sub_rn(t1, t2);
                sum = add_rn(sum, mul_rn((float)ab.qs[sb * 32 + j], t3));
            }
        out = add_rn(out, mul_rn(ab.d, sum));
    }
    c[idx] = out;
}

__constant__ uint16_t kIq2GridCodes[256] = PFNG_IQ2XXS_GRID_CODES_INIT;

__device__ __forceinline__ int iq2_magnitude(unsigned entry, unsigned j) {
    const unsigned code = (kIq2GridCodes[entry] >> (2 * j)) & 3u;
    return code == 0 ? 8 : (code == 1 ? 25 : 43);
}

// llama_reference.cpp:148-161 with kernels/common/iq2_xxs.h:29-41 decode
__global__ void naive_iq2_xxs_kernel(const pfng_block_iq2_xxs *__restrict__ w, const pfng_block_q8_K *__restrict__ a,
                                     float *__restrict__ c, int64_t m, int64_t n, int64_t nb) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= m * n) return;
    const int64_t mi = idx / n, ni = idx % n;
    float out = 0.0f;
    for (int64_t b = 0; b < nb; ++b) {
        const pfng_block_iq2_xxs &wb = w[ni * nb + b];
        const pfng_block_q8_K &ab = a[mi * nb + b];
        const uint8_t *packed = reinterpret_cast<const uint8_t *>(wb.qs);
        int32_t sum = 0;
        for (int sb = 0; sb < 8; ++sb) {
            const uint8_t *p = packed + sb * 8;
            const uint32_t sas = (uint32_t)p[4] | ((uint32_t)p[5] << 8) | ((uint32_t)p[6] << 16) | ((uint32_t)p[7] << 24);
            int32_t s = 0;
            for (int g = 0; g < 4; ++g) {
                const unsigned index = (sas >> (7 * g)) & 0x7f;
                const unsigned signs = index | ((unsigned)__builtin_parity(index) << 7);
                for (int l = 0; l < 8; ++l) {
                    const int mag = iq2_magnitude(p[g], l);
                    const int v = (signs & (1u << l)) ? -mag : mag;
                    s += v * ab.qs[sb * 32 + g * 8 + l];
                }
            }
            sum += (2 * (int)((sas >> 28) & 15) + 1) * s;
        }
        const float t0 = mul_rn(0.125f, fp16_to_f32(wb.d));
        const float t1 = mul_rn(t0, ab.d);
        out = add_rn(out, mul_rn(t1, (float)sum));
    }
    c[idx] = out;
}

}  // namespace

hipError_t launch_naive_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                                hipStream_t stream) {
    const int64_t total = m * n;
    if (total == 0) return hipSuccess;
    const dim3 grid((unsigned)((total + 255) / 256)), block(256);
    switch (type) {
    case PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0:
        hipLaunchKernelGGL(naive_q4_0_kernel, grid, block, 0, stream, static_cast<const pfng_block_q4_0 *>(w),
                           static_cast<const pfng_block_q8_0 *>(a), c, m, n, k / 32);
        break;
    case PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K:
        hipLaunchKernelGGL(naive_q4_K_kernel, grid, block, 0, stream, static_cast<const pfng_block_q4_K *>(w),
                           static_cast<const pfng_block_q8_K *>(a), c, m, n, k / 256);
        break;
    case PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K:
        hipLaunchKernelGGL(naive_iq2_xxs_kernel, grid, block, 0, stream, static_cast<const pfng_block_iq2_xxs *>(w),
                           static_cast<const pfng_block_q8_K *>(a), c, m, n, k / 256);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace pfng
