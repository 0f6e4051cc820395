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

// (int)roundf(t), half away from zero, for the |t| <= 130 the q8 quantizers
// produce (|x * id| <= 127 up to rounding; an infinite id gives +-inf or NaN,
// which take the same conversion either way): trunc(t + copysign(0.5 - 2^-25,
// t)) in three operations instead of roundf's six. Equal to roundf for every
// float in [0, 130] (checked exhaustively), and both sides are odd functions.
__device__ __forceinline__ int round_half_away_q8(float t) {
    return (int)add_rn(t, __builtin_copysignf(0x1.fffffep-2f, t));
}

// Four values of a q8_0 / q8_K block: (int8)round(x * id) packed little-endian
// (llama_reference.cpp:49, :63; x * id separately rounded, roundf = std::round).
__device__ __forceinline__ uint32_t q8_quantize4(float4 v, float id) {
    const int q0 = round_half_away_q8(mul_rn(v.x, id));
    const int q1 = round_half_away_q8(mul_rn(v.y, id));
    const int q2 = round_half_away_q8(mul_rn(v.z, id));
    const int q3 = round_half_away_q8(mul_rn(v.w, id));
    return (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
           ((uint32_t)(q3 & 0xff) << 24);
}

// Butterfly reductions inside groups of W lanes (W a power of two <= 64).

// largest power of two <= v for v in 1..16, and the log2 of a power of two
constexpr int pow2_floor16(int v) { return v >= 16 ? 16 : (v >= 8 ? 8 : (v >= 4 ? 4 : (v >= 2 ? 2 : 1))); }
constexpr int log2_pow2(int v) { return v == 16 ? 4 : (v == 8 ? 3 : (v == 4 ? 2 : (v == 2 ? 1 : 0))); }
constexpr int pow2_ceil16(int v) { return v <= 1 ? 1 : (v <= 2 ? 2 : (v <= 4 ? 4 : (v <= 8 ? 8 : 16))); }


// Sums over aligned groups of G lanes with DPP adds: two quad permutes, the
// half-row and row mirrors, then the gfx9 family's row_bcast:15 and
// row_bcast:31. One VALU add per step, no LDS permute. For G <= 16 every lane
// of a group ends with the group's sum; for G = 32 and 64 the group's last
// lane does (the others hold partial sums). Every lane must be active.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_src(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}
template <int G>
__device__ __forceinline__ float group_sum_dpp(float v) {
    static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group of 4..64 lanes");
    auto add = [](float x, int t) { return x + __builtin_bit_cast(float, t); };
    v = add(v, dpp_src<0xB1, 0xf>(__builtin_bit_cast(int, v)));       // quad_perm [1,0,3,2]
    v = add(v, dpp_src<0x4E, 0xf>(__builtin_bit_cast(int, v)));       // quad_perm [2,3,0,1]
    if constexpr (G >= 8) v = add(v, dpp_src<0x141, 0xf>(__builtin_bit_cast(int, v)));  // row_half_mirror
    if constexpr (G >= 16) v = add(v, dpp_src<0x140, 0xf>(__builtin_bit_cast(int, v))); // row_mirror
    if constexpr (G >= 32) v = add(v, dpp_src<0x142, 0xa>(__builtin_bit_cast(int, v))); // row_bcast:15
    if constexpr (G >= 64) v = add(v, dpp_src<0x143, 0xc>(__builtin_bit_cast(int, v))); // row_bcast:31
    return v;
}
template <int G>
__device__ __forceinline__ int group_sum_dpp(int v) {
    static_assert(G == 4 || G == 8 || G == 16, "integer groups of 4..16 lanes");
    v += dpp_src<0xB1, 0xf>(v);
    v += dpp_src<0x4E, 0xf>(v);
    if constexpr (G >= 8) v += dpp_src<0x141, 0xf>(v);
    if constexpr (G >= 16) v += dpp_src<0x140, 0xf>(v);
    return v;
}
__device__ __forceinline__ float wave_sum_lane63(float v) { return group_sum_dpp<64>(v); }

// v of lane (lane ^ O), O a power of two below 64, with the cheapest exact
// exchange: DPP quad permutes for 1 and 2, ds_swizzle's bit-mask mode for 4,
// 8 and 16 (within 32 lanes), ds_bpermute for 32.
template <int O>
__device__ __forceinline__ int xor_shfl(int v) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8 || O == 16 || O == 32, "xor offset");
    if constexpr (O == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
    else if constexpr (O == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
    else if constexpr (O <= 16) return __builtin_amdgcn_ds_swizzle(v, (O << 10) | 0x1f);
    else return __shfl_xor(v, O, 64);
}
template <int O>
__device__ __forceinline__ float xor_shfl(float v) {
    return __builtin_bit_cast(float, xor_shfl<O>(__builtin_bit_cast(int, v)));
}

// Butterfly over aligned groups of W lanes (exchange offsets W/2, ..., 1):
// every lane ends with op over its group, combined in the same pairs and
// order as a __shfl_xor loop, through xor_shfl's cheaper exchanges.
template <int O, class T, class Op>
__device__ __forceinline__ T butterfly(T v, Op op) {
    v = op(v, xor_shfl<O>(v));
    if constexpr (O > 1) return butterfly<O / 2>(v, op);
    else return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
    return butterfly<W / 2>(v, [](float a, float b) { return fmaxf(a, b); });
}
template <int W>
__device__ __forceinline__ int group_sum(int v) {
    return butterfly<W / 2>(v, [](int a, int b) { return a + b; });
}

// One lane's share of a q8_K super-block (llama_reference.cpp:54-70) when a
// wavefront quantizes one block, lane l owning elements 4l..4l+3: its four
// qs bytes, the block's d, and (valid on lanes 4i) bsums[i] = the sum of
// elements 16i..16i+15. The quantize kernel and the fused GEMVs share it, so
// their bytes are the same.
struct Q8KLane {
    uint32_t q;
    int bsum;
    float d;
};
__device__ __forceinline__ Q8KLane q8_K_quantize_lane(float4 v) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = group_max<64>(amax);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint32_t q = q8_quantize4(v, id);
    int s = (int)(int8_t)(q & 0xff) + (int)(int8_t)((q >> 8) & 0xff) + (int)(int8_t)((q >> 16) & 0xff) +
            (int)(int8_t)(q >> 24);
    s = group_sum<4>(s);
    return {q, s, d};
}

// Stores a lane's share into a 292-byte q8_K block (global or LDS).
__device__ __forceinline__ void q8_K_store_lane(uint8_t *out, const Q8KLane &r, int lane) {
    reinterpret_cast<uint32_t *>(out + 4)[lane] = r.q;
    if ((lane & 3) == 0) reinterpret_cast<int16_t *>(out + 260)[lane >> 2] = (int16_t)r.bsum;
    if (lane == 0) *reinterpret_cast<float *>(out) = r.d;
}

template <int W>
__device__ __forceinline__ float group_sumf(float v) {
    return butterfly<W / 2>(v, [](float a, float b) { return a + b; });
}

// Reduce-scatter exchanges: x[i] += x[i + H] of lane (lane ^ O) for i < H,
// then H/2 with O/2, down to H = 1. A lane whose O bit is clear keeps the
// lower half; callers lay out their values so that every lane keeps the lower
// half and sends the upper (lane-dependent rows, constant indices).
template <int H, int O, int BASE = 0, class T, int N>
__device__ __forceinline__ void reduce_scatter_steps(T (&x)[N]) {
    static_assert(H >= 1 && BASE + 2 * H <= N, "halves within the array");
#pragma unroll
    for (int i = 0; i < H; ++i) x[BASE + i] += xor_shfl<O>(x[BASE + i + H]);
    if constexpr (H > 1) reduce_scatter_steps<H / 2, O / 2, BASE>(x);
}


// D(32x32, int32) = A(32x32 int8) . B(32x32 int8)^T + C.
// Operand lane l supplies row (l % 32) with the 16 bytes of K-half (l / 32);
// A and B use the same K mapping, so any per-half byte order that is the same
// on both sides yields the full 32-term dot product.
// Result lane l, register r holds row 8*(r/4) + 4*(l/32) + (r%4), column l%32.
__device__ __forceinline__ i32x16 mfma_i8_32x32x32(i32x4 a, i32x4 b, i32x16 c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// D(16x16, int32) = A(16x32 int8) . B(16x32 int8)^T + C.
// Operand lane l supplies row (l % 16) with the 8 bytes of K-quarter (l / 16);
// A and B use the same K mapping, so any assignment of the 32 K positions to
// (quarter, byte) that is the same on both sides yields the full dot product.
// Result lane l, register r holds row 4*(l/16) + r, column l%16.
__device__ __forceinline__ i32x4 mfma_i8_16x16x32(uint64_t a, uint64_t b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, c, 0, 0, 0);
}

// D(32x32, fp32) = A(32x8 fp16) . B(32x8 fp16)^T + C, same result layout.
__device__ __forceinline__ f32x16 mfma_f16_32x32x8(f16x4 a, f16x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, c, 0, 0, 0);
}

// D(32x32, fp32) = A(32x16 fp16) . B(32x16 fp16)^T + C, same result layout.
__device__ __forceinline__ f32x16 mfma_f16_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// q4_K scale and min of sub-block j (0..7) from the 12 packed bytes (hd[1..3];
// hd[0] holds d and dmin), with the reference's decode
// (llama_reference.cpp:116-121).
__device__ __forceinline__ void q4_K_scale_min(const uint32_t hd[4], int j, uint32_t &sc, uint32_t &mn) {
    auto byte = [&](int i) { return (hd[1 + i / 4] >> (8 * (i % 4))) & 0xffu; };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 15) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// An output element stored with system scope (a relaxed atomic store:
// global_store with sc0 sc1), so it is written through L2 to memory. The
// GEMM tiles and the chunked tile GEMVs do not read their output again, and
// a kernel's end then finds no dirty output lines in L2 to write back
// (480x1536x1536: 7.41 -> 7.19 us against non-temporal stores, 128-row
// decode batches 15.8 -> 15.6 us). Not for the one-float-per-row stores of
// the M = 1 GEMVs, which lose L2's write combining (c1 3.71 -> 3.85 us).
__device__ __forceinline__ void store_through(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void store_through(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// Bytes of v (each 0..15) times the digit in both 16-bit halves of digit2
// (0..7): one packed 16-bit multiply per dword, and no byte product (<= 105)
// carries into the next byte.
__device__ __forceinline__ i32x4 mul_planes(i32x4 v, uint32_t digit2) {
    i32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u16x2 x = __builtin_bit_cast(u16x2, (uint32_t)v[i]) * __builtin_bit_cast(u16x2, digit2);
        o[i] = (int32_t)__builtin_bit_cast(uint32_t, x);
    }
    return o;
}

// XCD-aware tile order for a 1-D grid of mt x nt output tiles. Workgroup ids
// are dealt round-robin to MI355X's 8 XCDs (id % 8), each with its own L2;
// regroup them so that each XCD owns a contiguous range of tiles, walked
// m-fastest in groups of kGroupM m-tiles, so the workgroups resident on one XCD
// at a time share weight and activation tiles in its L2. The map is a bijection
// on [0, mt*nt): the first 8*q ids are regrouped (q tiles per XCD), the last
// (mt*nt) % 8 ids keep their own index. kGroupM = 1 walks n fastest, so an
// XCD's range covers as few m-tiles (activation rows) as possible.
struct TileOrigin {
    int mi, ni;  // tile coordinates
};
template <int kGroupM = 8>
__device__ __forceinline__ TileOrigin xcd_tile(int id, int mt, int nt) {
    constexpr int kXcds = 8;
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

// Q4_0 nibbles of one qs dword -> 16 * (nibble - 8) as packed int8, for the
// bytes kMask keeps (0xF0 per byte kept, 0x00 per byte zeroed). With the
// nibble q in the upper half of a byte, the byte is 16 * q; flipping its top
// bit subtracts 128 modulo 256, which read as int8 is 16 * (q - 8) for every
// q, with no carries between bytes. Each is a shift (low nibbles only) and
// one and-xor (v_bitop3).
template <uint32_t kMask = 0xF0F0F0F0u>
__device__ __forceinline__ uint32_t q4_0_lo16(uint32_t x) {
    return ((x << 4) & kMask) ^ (kMask & 0x80808080u);
}
template <uint32_t kMask = 0xF0F0F0F0u>
__device__ __forceinline__ uint32_t q4_0_hi16(uint32_t x) {
    return (x & kMask) ^ (kMask & 0x80808080u);
}
__device__ __forceinline__ void q4_0_unpack16(uint32_t x, uint32_t &lo16, uint32_t &hi16) {
    lo16 = q4_0_lo16(x);
    hi16 = q4_0_hi16(x);
}

// Marks the N registers of x as used at this point: the loads that produce
// them can then not be sunk below it (into a later branch that is the only
// other user, say), and the compiler waits for exactly those loads here.
template <int N>
__device__ __forceinline__ void use_here(const uint32_t (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" ::"v"(x[i]));
}

// Marks the N registers of x as redefined at this point: nothing computed
// from them can be moved above it (arithmetic on loaded values hoisted above
// a workgroup barrier makes the barrier wait for those loads).
template <class T, int N>
__device__ __forceinline__ void redefine_here(T (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(x[i]));
}

// dw * da of two fp16 scales (the low or high halves of a and b) in fp32: the
// product of two fp16 values is exact in fp32, so this equals
// fp16_to_f32(dw) * fp16_to_f32(da) and compiles to one mixed-precision fma.
template <bool kAHi, bool kBHi>
__device__ __forceinline__ float fp16_product(uint32_t a, uint32_t b) {
    const _Float16 ha = __builtin_bit_cast(_Float16, (uint16_t)(kAHi ? a >> 16 : a));
    const _Float16 hb = __builtin_bit_cast(_Float16, (uint16_t)(kBHi ? b >> 16 : b));
    return __builtin_fmaf((float)ha, (float)hb, 0.0f);
}

// One flat run of kRows x kCols 16-byte chunks into LDS at dst with direct
// loads: chunk (r, j) from src + r * rstride + 16 (col0 + j), 64 chunks per
// instruction (1 KB at dst + 1024 i), every lane active: lanes past the end
// repeat the last chunk into the pad that follows the run, and rows at or past
// rvalid repeat row rvalid - 1. (A copy whose lanes are predicated may be
// merged by the compiler into one whose LDS address comes from a single lane.)
template <int kRows, int kCols>
__device__ __forceinline__ void run_copy(const uint8_t *src, uint32_t rstride, int col0, int rvalid, uint8_t *dst,
                                         int lane) {
    constexpr int kN = kRows * kCols;
#pragma unroll
    for (int i = 0; i < (kN + 63) / 64; ++i) {
        int p = 64 * i + lane;
        if (p > kN - 1) p = kN - 1;
        int r = p / kCols;
        const int col = col0 + p - r * kCols;
        if (r > rvalid - 1) r = rvalid - 1;
        const uint32_t off = (uint32_t)r * rstride + 16u * (uint32_t)col;  // one 32-bit offset from a uniform base
        __builtin_amdgcn_global_load_lds(src + off, (__attribute__((address_space(3))) void *)(dst + i * 1024), 16,
                                         0, 0);
    }
}
// run_copy without the pad: the run's first kN / 64 * 64 chunks as above,
// the kN % 64 == 16 chunks left by one 4-byte copy (lane l: dword l % 4 of
// chunk kN / 64 * 64 + l / 4), so exactly kN * 16 bytes are written, every
// lane active, and in as many instructions as run_copy issues.
template <int kRows, int kCols>
__device__ __forceinline__ void run_copy_exact(const uint8_t *src, uint32_t rstride, int col0, int rvalid,
                                               uint8_t *dst, int lane) {
    constexpr int kN = kRows * kCols, kFull = kN / 64;
    static_assert(kN % 64 == 16, "a 16-chunk tail: one 4-byte copy of 64 lanes");
#pragma unroll
    for (int i = 0; i < kFull; ++i) {
        const int p = 64 * i + lane;
        int r = p / kCols;
        const int col = col0 + p - r * kCols;
        if (r > rvalid - 1) r = rvalid - 1;
        const uint32_t off = (uint32_t)r * rstride + 16u * (uint32_t)col;
        __builtin_amdgcn_global_load_lds(src + off, (__attribute__((address_space(3))) void *)(dst + i * 1024), 16,
                                         0, 0);
    }
    const int p = 64 * kFull + (lane >> 2);
    int r = p / kCols;
    const int col = col0 + p - r * kCols;
    if (r > rvalid - 1) r = rvalid - 1;
    const uint32_t off = (uint32_t)r * rstride + 16u * (uint32_t)col + 4u * (uint32_t)(lane & 3);
    __builtin_amdgcn_global_load_lds(src + off, (__attribute__((address_space(3))) void *)(dst + kFull * 1024), 4, 0,
                                     0);
}
// The tile GEMVs' runs with C chunks of activation rows: without pad from two
// chunks on (a quarter fewer bytes copied: q4_0 4096 x 4096, m = 32 6.93 ->
// 6.77 us), with it at one chunk (m <= 16 measured 0.02 us slower without).
template <int C, int kRows, int kCols>
__device__ __forceinline__ void copy_run(const uint8_t *src, uint32_t rstride, int col0, int rvalid, uint8_t *dst,
                                         int lane) {
    if constexpr (C > 1)
        run_copy_exact<kRows, kCols>(src, rstride, col0, rvalid, dst, lane);
    else
        run_copy<kRows, kCols>(src, rstride, col0, rvalid, dst, lane);
}
// chunks of 16 activation rows the chunked MFMA tile GEMVs take (m <= 128)
constexpr int kMaxGemvChunks = 8;

// Largest m the chunked MFMA tile GEMVs take at this k: every chunk count from
// k = 2048; below it, where the MFMA GEMM tiles are cheaper past four chunks
// (q4_0 k = 1024, m = 128: 10.44 us against 7.24), m = 64.
inline int gemv_tiles_max_m(int64_t k) { return k >= 2048 ? 16 * kMaxGemvChunks : 64; }

// instructions (1-KB pieces) of a run_copy run
template <int kRows, int kCols>
__host__ __device__ constexpr int run_copies() {
    return (kRows * kCols + 63) / 64;
}

}  // namespace pfng
