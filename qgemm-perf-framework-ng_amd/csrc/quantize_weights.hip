// Weight quantizers for gfx950: q4_0 and q4_K, byte-identical to the
// reference's host quantizers llama_reference::quantize_row_q4_0 and
// quantize_row_q4_K (bench/llama_reference/llama_reference.cpp:13-36, 72-111),
// including q4_K's non-upstream scale packing. They are setup kernels: fast
// generation of large weight matrices on the device; the benchmarked paths
// take weights in the reference's byte layout whichever side produced them.
//
// Bit-exactness relies on the same rules as the activation quantizers
// (separately rounded fp32 steps, correctly rounded division, roundf = half
// away from zero, the ggml fp32 -> fp16 routine) plus:
//   * q4_0's scale comes from the first element of largest magnitude (the
//     reference's strict "<" scan), which a lane-parallel reduction keeps by
//     ordering candidates by (|x|, lowest index);
//   * float -> int conversions of values outside the int32 range return
//     INT_MIN, as the reference's x86-64 build does (cvttss2si); they can only
//     occur for degenerate sub-blocks (range far below the offset).
#include <climits>

#include "device_common.h"
#include "kernels.h"

namespace pfng {

namespace {

__device__ __forceinline__ int cvt_i32_x86(float v) {
    return (v >= -2147483648.0f && v < 2147483648.0f) ? (int)v : INT_MIN;
}

// 8 lanes per 32-value block, 32 blocks per 256-thread workgroup.
__global__ __launch_bounds__(256) void quantize_q4_0_kernel(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                           int64_t nblocks) {
    const int sub = threadIdx.x & 7;
    const int64_t block = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool valid = block < nblocks;
    float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) v4 = *reinterpret_cast<const float4 *>(x + block * 32 + sub * 4);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    // first element of largest magnitude: key = (|x| bits, 255 - index);
    // a lane with no element above 0 keeps key 0 and the reference's initial 0
    uint32_t kbits = 0, kidx = 0;
    float smax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float av = fabsf(v[i]);
        if (__builtin_bit_cast(float, kbits) < av) {
            kbits = f32_bits(av);
            kidx = 255u - (uint32_t)(sub * 4 + i);
            smax = v[i];
        }
    }
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) {
        const uint32_t ob = __shfl_xor(kbits, o, kWave), oi = __shfl_xor(kidx, o, kWave);
        const float os = __shfl_xor(smax, o, kWave);
        if (ob > kbits || (ob == kbits && oi > kidx)) {
            kbits = ob;
            kidx = oi;
            smax = os;
        }
    }
    const float d = smax / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = (int)(int8_t)(int)add_rn(mul_rn(v[i], id), 8.5f);
        q[i] = t < 15 ? t : 15;
    }
    // byte i of qs = q_i | q_(i+16) << 4: lanes 0..3 hold i = 0..15, lanes 4..7 the partners
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int hi = __shfl_down(q[i], 4, 8);
        packed |= (uint32_t)((q[i] & 15) | ((hi & 15) << 4)) << (8 * i);
    }
    if (valid && sub < 4) {
        uint16_t *out = reinterpret_cast<uint16_t *>(y + block * 18 + 2 + 4 * sub);
        out[0] = (uint16_t)(packed & 0xffffu);
        out[1] = (uint16_t)(packed >> 16);
        if (sub == 0) *reinterpret_cast<uint16_t *>(y + block * 18) = (uint16_t)f32_to_fp16_bits(d);
    }
}

// One wavefront per 256-value super-block; lane l owns values 4l..4l+3 of
// sub-block l / 8.
__global__ __launch_bounds__(256) void quantize_q4_K_kernel(const float *__restrict__ x, uint8_t *__restrict__ y,
                                                           int64_t nblocks) {
    const int lane = threadIdx.x & 63;
    const int64_t block = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (block >= nblocks) return;  // whole wave leaves together
    const float4 v4 = *reinterpret_cast<const float4 *>(x + block * 256 + lane * 4);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    float lo = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
    float hi = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, o, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, o, kWave));
    }
    const float ls = sub_rn(hi, lo) / 15.0f;
    const float lm = -lo / (ls != 0.0f ? ls : 1.0f);
    // block maxima start from 0, as in the reference
    float maxs = fmaxf(ls, 0.0f), maxm = fmaxf(lm, 0.0f);
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) {
        maxs = fmaxf(maxs, __shfl_xor(maxs, o, kWave));
        maxm = fmaxf(maxm, __shfl_xor(maxm, o, kWave));
    }
    const float ds = maxs / 63.0f, dm = maxm / 63.0f;
    const int si = cvt_i32_x86(roundf(ls / (ds != 0.0f ? ds : 1.0f)));
    const int mi = cvt_i32_x86(roundf(lm / (dm != 0.0f ? dm : 1.0f)));
    const uint32_t s8 = (uint32_t)(si < 63 ? si : 63) & 0xffu;  // uint8_t s[i] = std::min(63, ...)
    const uint32_t m8 = (uint32_t)(mi < 63 ? mi : 63) & 0xffu;
    // values: clamp(round(x / ls + lm), 0, 15)
    const float div = ls != 0.0f ? ls : 1.0f;
    uint32_t qv = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int t = cvt_i32_x86(roundf(add_rn(v[i] / div, lm)));
        t = t < 0 ? 0 : (t > 15 ? 15 : t);
        qv |= (uint32_t)t << (8 * i);
    }
    // qs[p*32 + j] = q(2p, j) | q(2p+1, j) << 4: the odd sub-block sits 8 lanes up
    const uint32_t partner = __shfl_down(qv, 8, kWave);
    uint8_t *blk = y + block * 144;
    const int sb = lane >> 3;
    if ((sb & 1) == 0)
        *reinterpret_cast<uint32_t *>(blk + 16 + (sb / 2) * 32 + 4 * (lane & 7)) = qv | (partner << 4);
    // header: d, dmin, 12 bytes of scales/mins with the reference's packing
    uint32_t s[8], m[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s[i] = __shfl(s8, 8 * i, kWave);
        m[i] = __shfl(m8, 8 * i, kWave);
    }
    if (lane == 0) {
        uint32_t sc[12];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = (s[i] | ((s[i + 4] & 3u) << 6)) & 0xffu;
            sc[i + 4] = (m[i] | ((m[i + 4] & 3u) << 6)) & 0xffu;
            sc[i + 8] = ((s[i + 4] >> 2) | ((m[i + 4] >> 2) << 4)) & 0xffu;
        }
        uint4 hd;
        hd.x = f32_to_fp16_bits(ds) | (f32_to_fp16_bits(dm) << 16);
        hd.y = sc[0] | (sc[1] << 8) | (sc[2] << 16) | (sc[3] << 24);
        hd.z = sc[4] | (sc[5] << 8) | (sc[6] << 16) | (sc[7] << 24);
        hd.w = sc[8] | (sc[9] << 8) | (sc[10] << 16) | (sc[11] << 24);
        *reinterpret_cast<uint4 *>(blk) = hd;
    }
}

}  // namespace

hipError_t launch_quantize_q4_0(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream) {
    const int64_t nblocks = rows * (k / 32);
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q4_0_kernel, dim3((unsigned)((nblocks + 31) / 32)), dim3(256), 0, stream, x,
                       static_cast<uint8_t *>(y), nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q4_K(const float *x, void *y, int64_t rows, int64_t k, hipStream_t stream) {
    const int64_t nblocks = rows * (k / 256);
    if (nblocks == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_q4_K_kernel, dim3((unsigned)((nblocks + 3) / 4)), dim3(256), 0, stream, x,
                       static_cast<uint8_t *>(y), nblocks);
    return hipGetLastError();
}

}  // namespace pfng
