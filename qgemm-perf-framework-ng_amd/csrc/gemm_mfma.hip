// int8-MFMA GEMM path for gfx950 (prefill-sized m).
//
// q4_0 x q8_0: C[m][n] = sum_b S_b[m][n] * da[m][b] * dw[n][b], with S_b the
// exact int32 dot of block b (llama_reference.cpp:134-146).
//
// Per workgroup tile BM x BN and per K stage of KB = 4 blocks (128 elements):
//   * global -> registers: each thread loads one 68-byte q8_0 block pair and
//     one 36-byte q4_0 block pair (4-byte aligned when k % 128 == 0), with the
//     loads of stage s+1 in flight while stage s is computed;
//   * registers -> LDS: activation int8 copied as is (realigned by 2 bytes for
//     the even block of a pair); weight nibbles expanded to 16*(q-8) int8;
//     padded 144-byte rows keep the 16-byte MFMA operand reads conflict free;
//   * per block and 32x32 tile: S16 = v_mfma_i32_32x32x32_i8(act, w16) (= 16*S_b),
//     P = v_mfma_f32_32x32x8_f16(da, dw) (= da*dw exactly, an outer product of
//     two fp16 vectors on the matrix core), acc = fma(float(S16), P, acc).
//     C = acc / 16 at the end (a power of two, so rounding is unaffected).
// The epilogue costs two VALU operations per (m, n, block) item (cvt + fma); the
// matrix core carries the scale products. This is the VALU-bound part of the
// format: the int8 MFMA itself would finish the same items about twice as fast.
//
// A diagnostic instantiation writes S_b instead of accumulating (block isums).
#include "device_common.h"
#include "kernels.h"

namespace pfng {

namespace {

constexpr int KB = 4;                     // blocks per K stage
constexpr int kRowStride = KB * 32 + 16;  // LDS bytes per tile row (int8 + pad)

template <int BM, int BN, int WM, int WN>
struct Q40Config {
    static constexpr int kBM = BM, kBN = BN, kWM = WM, kWN = WN;
    static constexpr int kThreads = 64 * WM * WN;
    static constexpr int TM = BM / WM / 32;  // 32x32 tiles per wave along m
    static constexpr int TN = BN / WN / 32;  // along n
    static constexpr int kActPairs = BM * KB / 2;
    static constexpr int kWPairs = BN * KB / 2;
    static constexpr int kActIters = (kActPairs + kThreads - 1) / kThreads;
    static constexpr int kWIters = (kWPairs + kThreads - 1) / kThreads;
    // LDS layout
    static constexpr int kAq = 0;
    static constexpr int kAd = kAq + BM * kRowStride;
    static constexpr int kWq = kAd + BM * KB * 2;
    static constexpr int kWd = kWq + BN * kRowStride;
    static constexpr int kZero = kWd + BN * KB * 8;
    static constexpr int kLdsBytes = kZero + 16;
    static_assert(TM >= 1 && TN >= 1, "tile too small");
};

struct ActRegs {
    uint32_t v[17];
};
struct WRegs {
    uint32_t v[9];
};

template <class C>
__device__ __forceinline__ void load_stage(const uint8_t *__restrict__ a, const uint8_t *__restrict__ w, int m, int n,
                                           int nb, int m0, int n0, int kb0, ActRegs (&ar)[C::kActIters],
                                           WRegs (&wr)[C::kWIters]) {
#pragma unroll
    for (int it = 0; it < C::kActIters; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        if (task < C::kActPairs) {
            const int r = task / (KB / 2), p = task % (KB / 2);
            int row = m0 + r;
            row = row < m ? row : m - 1;
            const uint32_t *src = reinterpret_cast<const uint32_t *>(a + ((size_t)row * nb + kb0 + 2 * p) * 34);
#pragma unroll
            for (int i = 0; i < 17; ++i) ar[it].v[i] = src[i];
        }
    }
#pragma unroll
    for (int it = 0; it < C::kWIters; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        if (task < C::kWPairs) {
            const int r = task / (KB / 2), p = task % (KB / 2);
            int row = n0 + r;
            row = row < n ? row : n - 1;
            const uint32_t *src = reinterpret_cast<const uint32_t *>(w + ((size_t)row * nb + kb0 + 2 * p) * 18);
#pragma unroll
            for (int i = 0; i < 9; ++i) wr[it].v[i] = src[i];
        }
    }
}

template <class C>
__device__ __forceinline__ void store_stage(uint8_t *lds, const ActRegs (&ar)[C::kActIters],
                                            const WRegs (&wr)[C::kWIters]) {
#pragma unroll
    for (int it = 0; it < C::kActIters; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        if (task < C::kActPairs) {
            const int r = task / (KB / 2), p = task % (KB / 2);
            const uint32_t *v = ar[it].v;
            uint4 *dst = reinterpret_cast<uint4 *>(lds + C::kAq + r * kRowStride + 2 * p * 32);
            dst[0] = make_uint4(shift2(v[0], v[1]), shift2(v[1], v[2]), shift2(v[2], v[3]), shift2(v[3], v[4]));
            dst[1] = make_uint4(shift2(v[4], v[5]), shift2(v[5], v[6]), shift2(v[6], v[7]), shift2(v[7], v[8]));
            dst[2] = make_uint4(v[9], v[10], v[11], v[12]);
            dst[3] = make_uint4(v[13], v[14], v[15], v[16]);
            *reinterpret_cast<uint32_t *>(lds + C::kAd + r * KB * 2 + 4 * p) = (v[0] & 0xffffu) | (v[8] & 0xffff0000u);
        }
    }
#pragma unroll
    for (int it = 0; it < C::kWIters; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        if (task < C::kWPairs) {
            const int r = task / (KB / 2), p = task % (KB / 2);
            const uint32_t *u = wr[it].v;
            uint32_t q0[4] = {shift2(u[0], u[1]), shift2(u[1], u[2]), shift2(u[2], u[3]), shift2(u[3], u[4])};
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q4_0_unpack16(q0[i], lo[i], hi[i]);
            uint4 *dst = reinterpret_cast<uint4 *>(lds + C::kWq + r * kRowStride + 2 * p * 32);
            dst[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            dst[1] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
            for (int i = 0; i < 4; ++i) q4_0_unpack16(u[5 + i], lo[i], hi[i]);
            dst[2] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            dst[3] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            // scale of block t placed in fp16 slot t of an 8-byte entry (slot-expanded)
            const uint32_t d0 = u[0] & 0xffffu, d1 = u[4] >> 16;
            uint2 *wd = reinterpret_cast<uint2 *>(lds + C::kWd + (r * KB + 2 * p) * 8);
            if (p == 0) {
                wd[0] = make_uint2(d0, 0u);
                wd[1] = make_uint2(d1 << 16, 0u);
            } else {
                wd[0] = make_uint2(0u, d0);
                wd[1] = make_uint2(0u, d1 << 16);
            }
        }
    }
}

// kIsums == false: fp32 C. kIsums == true: int32 block sums (diagnostic).
template <class C, bool kIsums>
__global__ __launch_bounds__(C::kThreads) void gemm_q4_0_kernel(const uint8_t *__restrict__ w,
                                                               const uint8_t *__restrict__ a, float *__restrict__ c,
                                                               int32_t *__restrict__ isums, int m, int n, int nb) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wave_m = wave / C::kWN;
    const int wave_n = wave % C::kWN;
    const int m0 = blockIdx.y * C::kBM;
    const int n0 = blockIdx.x * C::kBN;
    const int li = lane & 31;  // operand row within a 32x32 tile
    const int lh = lane >> 5;  // K half of the operand

    if (threadIdx.x < 4) reinterpret_cast<uint32_t *>(lds + C::kZero)[threadIdx.x] = 0u;

    f32x16 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = (f32x16){};

    ActRegs ar[C::kActIters];
    WRegs wr[C::kWIters];
    load_stage<C>(a, w, m, n, nb, m0, n0, 0, ar, wr);

    const int stages = nb / KB;
    for (int s = 0; s < stages; ++s) {
        __syncthreads();
        store_stage<C>(lds, ar, wr);
        __syncthreads();
        if (s + 1 < stages) load_stage<C>(a, w, m, n, nb, m0, n0, (s + 1) * KB, ar, wr);

        // per-stage activation scales: da of blocks 0..3 in the four fp16 slots
        f16x4 ad[C::TM];
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm) {
            const int r = wave_m * C::TM * 32 + tm * 32 + li;
            ad[tm] = *reinterpret_cast<const f16x4 *>(lds + C::kAd + r * KB * 2);
        }
#pragma unroll
        for (int t = 0; t < KB; ++t) {
            i32x4 av[C::TM], wv[C::TN];
            f16x4 wd[C::TN];
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm) {
                const int r = wave_m * C::TM * 32 + tm * 32 + li;
                av[tm] = *reinterpret_cast<const i32x4 *>(lds + C::kAq + r * kRowStride + t * 32 + lh * 16);
            }
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const int r = wave_n * C::TN * 32 + tn * 32 + li;
                wv[tn] = *reinterpret_cast<const i32x4 *>(lds + C::kWq + r * kRowStride + t * 32 + lh * 16);
                const int off = lh ? C::kZero : C::kWd + (r * KB + t) * 8;
                wd[tn] = *reinterpret_cast<const f16x4 *>(lds + off);
            }
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < C::TN; ++tn) {
                    const i32x16 s16 = mfma_i8_32x32x32(av[tm], wv[tn], (i32x16){});
                    if constexpr (kIsums) {
                        const int col = n0 + wave_n * C::TN * 32 + tn * 32 + li;
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int row = m0 + wave_m * C::TM * 32 + tm * 32 + mfma_row(lane, r);
                            if (row < m && col < n) isums[((size_t)row * n + col) * nb + s * KB + t] = s16[r] / 16;
                        }
                    } else {
                        const f32x16 p = mfma_f16_32x32x8(ad[tm], wd[tn], (f32x16){});
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[tm][tn][r] = fmaf((float)s16[r], p[r], acc[tm][tn][r]);
                    }
                }
        }
    }

    if constexpr (!kIsums) {
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const int col = n0 + wave_n * C::TN * 32 + tn * 32 + li;
                if (col < n) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wave_m * C::TM * 32 + tm * 32 + mfma_row(lane, r);
                        if (row < m) c[(size_t)row * n + col] = acc[tm][tn][r] * 0.0625f;
                    }
                }
            }
    }
}

template <class C, bool kIsums>
hipError_t launch_q4_0(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n, int64_t k,
                       hipStream_t stream) {
    const dim3 grid((unsigned)((n + C::kBN - 1) / C::kBN), (unsigned)((m + C::kBM - 1) / C::kBM));
    hipLaunchKernelGGL((gemm_q4_0_kernel<C, kIsums>), grid, dim3(C::kThreads), C::kLdsBytes, stream,
                       static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, isums, (int)m, (int)n,
                       (int)(k / 32));
    return hipGetLastError();
}

using Q40Big = Q40Config<128, 128, 2, 2>;
using Q40Small = Q40Config<64, 64, 2, 2>;

}  // namespace

bool mfma_supported(int type, int64_t m, int64_t k) {
    (void)m;
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return k % (32 * KB) == 0;
    return false;
}

hipError_t launch_mfma_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                               hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return hipErrorInvalidValue;
    const int64_t big_tiles = ((m + 127) / 128) * ((n + 127) / 128);
    if (big_tiles >= 512) return launch_q4_0<Q40Big, false>(w, a, c, nullptr, m, n, k, stream);
    return launch_q4_0<Q40Small, false>(w, a, c, nullptr, m, n, k, stream);
}

hipError_t launch_mfma_block_isums(int type, const void *w, const void *a, int32_t *out, int64_t m, int64_t n,
                                   int64_t k, hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return hipErrorInvalidValue;
    return launch_q4_0<Q40Small, true>(w, a, nullptr, out, m, n, k, stream);
}

}  // namespace pfng
