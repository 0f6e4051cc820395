// Device helpers shared by the gfx950 kernels: vector types, fp16 bit
// conversions, wave reductions and the MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pfng_blocks.h"

namespace pfng {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Separately rounded fp32 operations. The operators are evaluated under
// "fp contract(off)" so the backend never fuses them into an FMA; the HIP
// header's __fmul_rn/__fadd_rn are compiled with contraction enabled and do
// get fused with neighbouring operations.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

__device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float f32_from(uint32_t u) { return __builtin_bit_cast(float, u); }

// Exact widening, as ggml_compute_fp16_to_fp32 (include/ggml.h:83-97) for every
// finite input, infinities and zeros (the hardware conversion is exact).
__device__ __forceinline__ float fp16_to_f32(uint32_t h16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// ggml_compute_fp32_to_fp16 (include/ggml.h:99-117) step for step, so that the
// scale bytes written by the quantizers match the reference for every input.
__device__ __forceinline__ uint32_t f32_to_fp16_bits(float value) {
    const float scale_to_inf = 0x1.0p+112f;
    const float scale_to_zero = 0x1.0p-110f;
    float base = mul_rn(mul_rn(fabsf(value), scale_to_inf), scale_to_zero);
    const uint32_t w = f32_bits(value);
    const uint32_t shl1_w = w + w;
    const uint32_t sign = w & 0x80000000u;
    uint32_t bias = shl1_w & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base = add_rn(f32_from((bias >> 1) + 0x07800000u), base);
    const uint32_t bits = f32_bits(base);
    const uint32_t exp_bits = (bits >> 13) & 0x00007C00u;
    const uint32_t mantissa_bits = bits & 0x00000FFFu;
    const uint32_t nonsign = exp_bits + mantissa_bits;
    return (sign >> 16) | (shl1_w > 0xFF000000u ? 0x7E00u : nonsign);
}

// Four values of a q8_0 / q8_K block: (int8)round(x * id) packed little-endian
// (llama_reference.cpp:49, :63; x * id separately rounded, roundf = std::round).
__device__ __forceinline__ uint32_t q8_quantize4(float4 v, float id) {
    const int q0 = (int)roundf(mul_rn(v.x, id));
    const int q1 = (int)roundf(mul_rn(v.y, id));
    const int q2 = (int)roundf(mul_rn(v.z, id));
    const int q3 = (int)roundf(mul_rn(v.w, id));
    return (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
           ((uint32_t)(q3 & 0xff) << 24);
}

// Butterfly reductions inside groups of W lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// largest power of two <= v for v in 1..16, and the log2 of a power of two
constexpr int pow2_floor16(int v) { return v >= 16 ? 16 : (v >= 8 ? 8 : (v >= 4 ? 4 : (v >= 2 ? 2 : 1))); }
constexpr int log2_pow2(int v) { return v == 16 ? 4 : (v == 8 ? 3 : (v == 4 ? 2 : (v == 2 ? 1 : 0))); }
constexpr int pow2_ceil16(int v) { return v <= 1 ? 1 : (v <= 2 ? 2 : (v <= 4 ? 4 : (v <= 8 ? 8 : 16))); }

template <int W>
__device__ __forceinline__ int group_sum(int v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

template <int W>
__device__ __forceinline__ float group_sumf(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// D(32x32, int32) = A(32x32 int8) . B(32x32 int8)^T + C.
// Operand lane l supplies row (l % 32) with the 16 bytes of K-half (l / 32);
// A and B use the same K mapping, so any per-half byte order that is the same
// on both sides yields the full 32-term dot product.
// Result lane l, register r holds row 8*(r/4) + 4*(l/32) + (r%4), column l%32.
__device__ __forceinline__ i32x16 mfma_i8_32x32x32(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// D(32x32, fp32) = A(32x8 fp16) . B(32x8 fp16)^T + C, same result layout.
__device__ __forceinline__ f32x16 mfma_f16_32x32x8(f16x4 a, f16x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, c, 0, 0, 0);
}

// D(32x32, fp32) = A(32x16 fp16) . B(32x16 fp16)^T + C, same result layout.
__device__ __forceinline__ f32x16 mfma_f16_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// XCD-aware tile order for a 1-D grid of mt x nt output tiles. Workgroup ids
// are dealt round-robin to MI355X's 8 XCDs (id % 8), each with its own L2;
// regroup them so that each XCD owns a contiguous range of tiles, walked
// m-fastest in groups of kGroupM m-tiles, so the workgroups resident on one XCD
// at a time share weight and activation tiles in its L2. The map is a bijection
// on [0, mt*nt): the first 8*q ids are regrouped (q tiles per XCD), the last
// (mt*nt) % 8 ids keep their own index.
struct TileOrigin {
    int mi, ni;  // tile coordinates
};
__device__ __forceinline__ TileOrigin xcd_tile(int id, int mt, int nt) {
    constexpr int kXcds = 8, kGroupM = 8;
    const int tiles = mt * nt;
    const int q = tiles / kXcds;
    const int t = id < q * kXcds ? (id % kXcds) * q + id / kXcds : id;
    const int gm = mt < kGroupM ? mt : kGroupM;
    const int group = t / (gm * nt), in = t % (gm * nt);
    const int gm_here = (mt - group * gm) < gm ? (mt - group * gm) : gm;
    return {group * gm + in % gm_here, in / gm_here};
}

// Row of result register r for lane l of a 32x32 MFMA tile.
__device__ __forceinline__ int mfma_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Bytes [2, 6) of the little-endian pair (lo, hi): realigns data that sits two
// bytes into a dword-aligned load.
__device__ __forceinline__ uint32_t shift2(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_alignbyte(hi, lo, 2);
}

// Q4_0 nibbles of one qs dword -> 16 * (nibble - 8) as packed int8.
// x ^ 0x88 flips bit 3 of each nibble, which turns (nibble - 8) into the same
// nibble read as a signed 4-bit number; placing it in the upper half of the
// byte yields 16 * (nibble - 8) with no carries between bytes.
__device__ __forceinline__ void q4_0_unpack16(uint32_t x, uint32_t &lo16, uint32_t &hi16) {
    const uint32_t y = x ^ 0x88888888u;
    lo16 = (y << 4) & 0xF0F0F0F0u;
    hi16 = y & 0xF0F0F0F0u;
}

}  // namespace pfng
