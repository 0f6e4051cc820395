// int8-MFMA GEMM path for gfx950 (prefill-sized m).
//
// q4_0 x q8_0: C[m][n] = sum_b S_b[m][n] * da[m][b] * dw[n][b], with S_b the
// exact int32 dot of block b (llama_reference.cpp:134-146).
//
// Workgroup tile BM x BN, K stages of KB blocks (32*KB elements):
//   * global -> registers: every thread loads whole q8_0 and q4_0 block pairs
//     (68 / 36 bytes, dword loads, 4-byte aligned when k % 64 == 0) one stage
//     ahead of the stage being computed. The loads are unconditional (rows
//     clamped at the matrix edge) and a scheduling barrier keeps them ahead of
//     the arithmetic.
//   * registers -> LDS: activation int8 copied (the even block of a pair
//     realigned by two bytes); weight nibbles expanded to 16*(q-8) int8; fp16
//     scales kept per row. Rows are padded so the 16-byte MFMA operand reads
//     are free of bank conflicts.
//   * per block and 32x32 tile: S16 = v_mfma_i32_32x32x32_i8(act, w16) (= 16*S_b),
//     P = v_mfma_f32_32x32x8_f16(da, dw) (the exact outer product da*dw on the
//     matrix core), acc = fma(float(S16), P, acc); C = acc / 16 at the end.
// The epilogue costs two VALU operations per (m, n, block) item; the int8
// matrix core finishes the same items about four times as fast (a wave64 VALU
// op takes 4 cycles, packed fp32 is not used), so this format is VALU-bound.
// Small problems use 32x32 tiles whose stage blocks are shared by two waves
// (their partial sums are added through LDS at the end), so that even a few
// hundred output tiles keep several waves resident on every CU.
//
// A diagnostic instantiation writes S_b instead of accumulating (block isums).
#include "device_common.h"
#include "kernels.h"

namespace pfng {

namespace {

// BM x BN workgroup tile, WM x WN waves over it, each wave's stage blocks
// divided among WK waves (WK > 1: the WK partial accumulators are added
// through LDS at the end, in wave order), KB q4_0 blocks per K stage.
// DEPTH register sets of loaded-but-not-stored stages: the loads of stage
// s+DEPTH+1 are issued while stage s is computed (deep prefetch for the small
// tiles, whose stages are too short to cover a memory round trip).
template <int BM, int BN, int WM, int WN, int KB, int WK = 1, int DEPTH = 1, int MINW = 2>
struct Q40Config {
    static constexpr int kBM = BM, kBN = BN, kWM = WM, kWN = WN, kKB = KB, kWK = WK, kDepth = DEPTH;
    // waves per SIMD the register budget must allow: the fp32 epilogue needs two
    // resident waves per SIMD to keep the VALU issuing while the other waits
    static constexpr int kMinWavesPerEU = MINW;
    static constexpr int kThreads = 64 * WM * WN * WK;
    static constexpr int kWaveBlocks = KB / WK;  // blocks per stage of one wave
    static constexpr int TM = BM / WM / 32;  // 32x32 tiles per wave along m
    static constexpr int TN = BN / WN / 32;  // along n
    static constexpr int kPairsPerRow = KB / 2;
    static constexpr int kActPairs = BM * kPairsPerRow;
    static constexpr int kWPairs = BN * kPairsPerRow;
    static constexpr int kActPT = kActPairs / kThreads;  // pairs per thread
    static constexpr int kWPT = kWPairs / kThreads;
    static constexpr int kRowStride = KB * 32 + 16;  // LDS bytes per tile row (int8 + pad)
    // LDS layout
    static constexpr int kAq = 0;
    static constexpr int kAd = kAq + BM * kRowStride;       // fp16 da[row][KB]
    static constexpr int kWq = kAd + BM * KB * 2;
    // dw[row][KB] as 32-bit words: block t's fp16 scale in the low half for
    // even t, in the high half for odd t, zeros in the other half
    static constexpr int kWd = kWq + BN * kRowStride;
    static constexpr int kBufBytes = kWd + BN * KB * 4;  // one stage
    // zeros that the upper K-half lanes read as their weight scale words
    static constexpr int kZero = 2 * kBufBytes;
    static constexpr int kZeroBytes = TN * 32 * KB * 4;
    static constexpr int kLdsBytes = kZero + kZeroBytes;  // double-buffered stages + zeros
    static_assert(TM >= 1 && TN >= 1, "tile too small");
    static_assert(KB % 4 == 0, "KB must be a multiple of 4 (scale vectors are read four at a time)");
    static_assert(kActPT * kThreads == kActPairs && kWPT * kThreads == kWPairs, "pairs must split evenly over threads");
    static_assert(kActPT >= 1 && kWPT >= 1, "every thread loads at least one pair of each operand");
    static_assert(kAd % 16 == 0 && kWq % 16 == 0 && kWd % 16 == 0, "LDS regions 16-byte aligned");
    static_assert(kWaveBlocks * WK == KB && kWaveBlocks % 4 == 0, "each wave takes a multiple of 4 blocks");
    static_assert((WK - 1) * WM * WN * TM * TN * 16 * 64 * 4 <= 2 * kBufBytes, "K-wave reduction fits in LDS");
    static_assert(kZeroBytes % 16 == 0 && kZeroBytes >= 16, "zero strip of whole 16-byte words");
};

template <class C>
struct StageRegs {
    uint32_t a[C::kActPT][17];
    uint32_t w[C::kWPT][9];
};

// Byte offsets of the block pairs a thread loads, from the workgroup's first
// row at the current stage's first block. They stay the same over the K loop
// (rows past the matrix edge are clamped to its last row), so each stage's
// loads are a uniform stage base plus these 32-bit offsets: no per-stage
// address arithmetic in the vector ALU. BM * nb * 34 < 2^32 for every k up to
// kMaxTiledK (mfma_supported declines longer rows).
template <class C>
struct LoadOffsets {
    uint32_t a[C::kActPT];
    uint32_t w[C::kWPT];
};

template <class C>
__device__ __forceinline__ LoadOffsets<C> load_offsets(int m, int n, int nb, int m0, int n0) {
    LoadOffsets<C> o;
#pragma unroll
    for (int it = 0; it < C::kActPT; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        const int row = m0 + task / C::kPairsPerRow;
        const int lrow = row < m ? row : m - 1;
        o.a[it] = ((uint32_t)(lrow - m0) * (uint32_t)nb + 2u * (uint32_t)(task % C::kPairsPerRow)) * 34u;
    }
#pragma unroll
    for (int it = 0; it < C::kWPT; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        const int row = n0 + task / C::kPairsPerRow;
        const int lrow = row < n ? row : n - 1;
        o.w[it] = ((uint32_t)(lrow - n0) * (uint32_t)nb + 2u * (uint32_t)(task % C::kPairsPerRow)) * 18u;
    }
    return o;
}

// a_st / w_st: the workgroup's first activation / weight row at the stage's
// first block (uniform across the workgroup).
template <class C>
__device__ __forceinline__ void load_stage(const uint8_t *a_st, const uint8_t *w_st, const LoadOffsets<C> &o,
                                           StageRegs<C> &r) {
#pragma unroll
    for (int it = 0; it < C::kActPT; ++it) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a_st + o.a[it]);
#pragma unroll
        for (int i = 0; i < 17; ++i) r.a[it][i] = src[i];
    }
#pragma unroll
    for (int it = 0; it < C::kWPT; ++it) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(w_st + o.w[it]);
#pragma unroll
        for (int i = 0; i < 9; ++i) r.w[it][i] = src[i];
    }
}

template <class C>
__device__ __forceinline__ void store_stage(uint8_t *lds, const StageRegs<C> &r) {
#pragma unroll
    for (int it = 0; it < C::kActPT; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        const int row = task / C::kPairsPerRow, p = task % C::kPairsPerRow;
        const uint32_t *v = r.a[it];
        uint4 *dst = reinterpret_cast<uint4 *>(lds + C::kAq + row * C::kRowStride + 2 * p * 32);
        dst[0] = make_uint4(shift2(v[0], v[1]), shift2(v[1], v[2]), shift2(v[2], v[3]), shift2(v[3], v[4]));
        dst[1] = make_uint4(shift2(v[4], v[5]), shift2(v[5], v[6]), shift2(v[6], v[7]), shift2(v[7], v[8]));
        dst[2] = make_uint4(v[9], v[10], v[11], v[12]);
        dst[3] = make_uint4(v[13], v[14], v[15], v[16]);
        *reinterpret_cast<uint32_t *>(lds + C::kAd + (row * C::kKB + 2 * p) * 2) = (v[0] & 0xffffu) | (v[8] & 0xffff0000u);
    }
#pragma unroll
    for (int it = 0; it < C::kWPT; ++it) {
        const int task = threadIdx.x + it * C::kThreads;
        const int row = task / C::kPairsPerRow, p = task % C::kPairsPerRow;
        const uint32_t *u = r.w[it];
        const uint32_t q0[4] = {shift2(u[0], u[1]), shift2(u[1], u[2]), shift2(u[2], u[3]), shift2(u[3], u[4])};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q4_0_unpack16(q0[i], lo[i], hi[i]);
        uint4 *dst = reinterpret_cast<uint4 *>(lds + C::kWq + row * C::kRowStride + 2 * p * 32);
        dst[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        dst[1] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
        for (int i = 0; i < 4; ++i) q4_0_unpack16(u[5 + i], lo[i], hi[i]);
        dst[2] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        dst[3] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *reinterpret_cast<uint2 *>(lds + C::kWd + (row * C::kKB + 2 * p) * 4) = make_uint2(u[0] & 0xffffu, u[4] & 0xffff0000u);
    }
}

// Operand fragments of one block t for the wave's TM x TN tiles. ad holds the
// da of blocks t4..t4+3 (t4 = t rounded down to a multiple of 4) in its four
// fp16 slots; wd holds dw of block t in slot t % 4 and zeros elsewhere, and
// the K-half 1 lanes read theirs from the zero strip, so the f16 MFMA of ad
// and wd is the exact outer product da * dw of block t.
template <class C>
struct Frags {
    i32x4 av[C::TM];
    i32x4 wv[C::TN];
    f16x4 ad[C::TM];
    f16x4 wd[C::TN];
};

// Per-lane LDS base addresses of one stage buffer; every fragment read is a
// base plus a compile-time offset (within the 16-bit ds_read immediate range).
struct FragBases {
    const uint8_t *aq, *ad, *wq, *wd;
};

template <class C>
__device__ __forceinline__ FragBases frag_bases(uint8_t *lds, int buf, int lane, int wave_m, int wave_n) {
    const int li = lane & 31, lh = lane >> 5;
    const int ra = wave_m * C::TM * 32 + li, rw = wave_n * C::TN * 32 + li;
    const uint8_t *b0 = lds + buf * C::kBufBytes;
    FragBases b;
    b.aq = b0 + C::kAq + ra * C::kRowStride + lh * 16;
    b.ad = b0 + C::kAd + ra * C::kKB * 2;
    b.wq = b0 + C::kWq + rw * C::kRowStride + lh * 16;
    b.wd = lh ? lds + C::kZero : b0 + C::kWd + rw * C::kKB * 4;
    return b;
}

// Fragments of block tb + j (tb a multiple of 4, j known at compile time).
template <class C>
__device__ __forceinline__ void load_frags(const FragBases &b, int tb, int j, Frags<C> &f) {
    const int t = tb + j, t4 = tb + (j & ~3);
#pragma unroll
    for (int tm = 0; tm < C::TM; ++tm) {
        f.av[tm] = *reinterpret_cast<const i32x4 *>(b.aq + tm * 32 * C::kRowStride + t * 32);
        f.ad[tm] = *reinterpret_cast<const f16x4 *>(b.ad + tm * 32 * C::kKB * 2 + t4 * 2);
    }
#pragma unroll
    for (int tn = 0; tn < C::TN; ++tn) {
        f.wv[tn] = *reinterpret_cast<const i32x4 *>(b.wq + tn * 32 * C::kRowStride + t * 32);
        const uint32_t word = *reinterpret_cast<const uint32_t *>(b.wd + tn * 32 * C::kKB * 4 + t * 4);
        f.wd[tn] = __builtin_bit_cast(f16x4, (j & 2) ? make_uint2(0u, word) : make_uint2(word, 0u));
    }
}

struct ItemRegs {
    i32x16 s16;
    f32x16 p;
};

// One K stage of one wave: its kWaveBlocks blocks (from tb) x TM x TN tiles
// = a flat list of items, software-pipelined so the MFMAs of item i+1 are in
// flight while the VALU epilogue of item i runs, and the LDS fragments of
// block t+1 load during block t.
template <class C, bool kIsums>
__device__ __forceinline__ void compute_stage(uint8_t *lds, int buf, f32x16 (&acc)[C::TM][C::TN], int32_t *isums,
                                              int m, int n, int nb, int m0, int n0, int s, int tb, int lane,
                                              int wave_m, int wave_n) {
    constexpr int kTiles = C::TM * C::TN;
    constexpr int kItems = C::kWaveBlocks * kTiles;
    // With several tiles per block, the fragments of block t+1 are read while
    // the items of block t run (two sets). With one tile per block there is no
    // such slack, so all of the stage's fragments are read up front.
    constexpr bool kAllFrags = kTiles == 1;
    constexpr int kSets = kAllFrags ? C::kWaveBlocks : 2;
    const FragBases bases = frag_bases<C>(lds, buf, lane, wave_m, wave_n);
    Frags<C> fr[kSets];
    ItemRegs it[2];
    if constexpr (kAllFrags) {
#pragma unroll
        for (int j = 0; j < C::kWaveBlocks; ++j) load_frags<C>(bases, tb, j, fr[j]);
    } else {
        load_frags<C>(bases, tb, 0, fr[0]);
    }
    auto issue = [&](int item) {
        const int t = item / kTiles, tile = item % kTiles;
        const int tm = tile / C::TN, tn = tile % C::TN;
        const Frags<C> &f = fr[kAllFrags ? t : (t & 1)];
        ItemRegs &r = it[item & 1];
        r.s16 = mfma_i8_32x32x32(f.av[tm], f.wv[tn], (i32x16){});
        if constexpr (!kIsums) r.p = mfma_f16_32x32x8(f.ad[tm], f.wd[tn], (f32x16){});
    };
    issue(0);
#pragma unroll
    for (int item = 0; item < kItems; ++item) {
        const int t = item / kTiles, tile = item % kTiles;
        const int tm = tile / C::TN, tn = tile % C::TN;
        if (!kAllFrags && tile == 0 && t + 1 < C::kWaveBlocks) load_frags<C>(bases, tb, t + 1, fr[(t + 1) & 1]);
        if (item + 1 < kItems) issue(item + 1);
        // keep the order: without the fences the scheduler sinks the MFMAs of
        // item+1 below this epilogue and reuses their result registers, which
        // exposes every MFMA's latency
        __builtin_amdgcn_sched_barrier(0);
        const ItemRegs &r = it[item & 1];
        if constexpr (kIsums) {
            const int col = n0 + wave_n * C::TN * 32 + tn * 32 + (lane & 31);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int row = m0 + wave_m * C::TM * 32 + tm * 32 + mfma_row(lane, q);
                if (row < m && col < n) isums[((size_t)row * n + col) * nb + s * C::kKB + tb + t] = r.s16[q] / 16;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[tm][tn][q] = fmaf((float)r.s16[q], r.p[q], acc[tm][tn][q]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// kIsums == false: fp32 C. kIsums == true: int32 block sums (diagnostic).
template <class C, bool kIsums>
__global__ __launch_bounds__(C::kThreads, C::kMinWavesPerEU) void gemm_q4_0_kernel(const uint8_t *__restrict__ w,
                                                                                  const uint8_t *__restrict__ a,
                                                                                  float *__restrict__ c,
                                                                                  int32_t *__restrict__ isums, int m,
                                                                                  int n, int nb) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wk = wave / (C::kWM * C::kWN);   // which share of each stage's blocks
    const int wmn = wave % (C::kWM * C::kWN);  // which TM x TN sub-tile
    const int wave_m = wmn / C::kWN;
    const int wave_n = wmn % C::kWN;
    const TileOrigin to = xcd_tile(blockIdx.x, (m + C::kBM - 1) / C::kBM, (n + C::kBN - 1) / C::kBN);
    const int m0 = to.mi * C::kBM, n0 = to.ni * C::kBN;
    const int li = lane & 31;  // operand row / result column within a 32x32 tile

    f32x16 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) acc[i][j] = (f32x16){};

    // Double-buffered LDS with one barrier per stage: stage s is computed from
    // one buffer while the registers of stage s+1 (loaded a stage earlier) are
    // stored into the other and the loads of stage s+2 are issued. Stores and
    // loads are unconditional (clamped stage index), so the loop body has no
    // divergent control flow.
    // regs[r] holds stage s+1 while stage s (s % kDepth == r) is computed.
    const int stages = nb / C::kKB;
    auto clampst = [&](int st) { return st < stages ? st : stages - 1; };
    // uniform row bases of the tile; stage st starts st * kKB blocks further
    const uint8_t *a_tile = a + (size_t)m0 * nb * 34;
    const uint8_t *w_tile = w + (size_t)n0 * nb * 18;
    const LoadOffsets<C> offs = load_offsets<C>(m, n, nb, m0, n0);
    for (int i = threadIdx.x; i < C::kZeroBytes / 16; i += C::kThreads)
        reinterpret_cast<uint4 *>(lds + C::kZero)[i] = make_uint4(0u, 0u, 0u, 0u);
    StageRegs<C> regs[C::kDepth];
    load_stage<C>(a_tile, w_tile, offs, regs[0]);
    store_stage<C>(lds, regs[0]);
#pragma unroll
    for (int r = 0; r < C::kDepth; ++r) {
        const int kb = clampst(1 + r) * C::kKB;
        load_stage<C>(a_tile + kb * 34, w_tile + kb * 18, offs, regs[r]);
    }
    __syncthreads();
    // The loop runs whole rounds of kRound stages (a multiple of kDepth and of
    // the two LDS buffers, so that register set and buffer are compile-time
    // constants and every fragment address is a base plus an immediate);
    // stages past the end skip only the arithmetic. Leaving the round with a
    // break instead made the compiler wait for freshly issued loads before
    // every barrier, which undid the prefetch.
    constexpr int kRound = C::kDepth % 2 == 0 ? C::kDepth : 2 * C::kDepth;
    for (int s0 = 0; s0 < stages; s0 += kRound) {
#pragma unroll
        for (int rr = 0; rr < kRound; ++rr) {
            const int s = s0 + rr;
            const int r = rr % C::kDepth;
            const int buf = rr & 1;
            __builtin_amdgcn_sched_barrier(0);
            if (s < stages)  // uniform across the workgroup
                compute_stage<C, kIsums>(lds, buf, acc, isums, m, n, nb, m0, n0, s, wk * C::kWaveBlocks, lane,
                                         wave_m, wave_n);
            __builtin_amdgcn_sched_barrier(0);
            store_stage<C>(lds + (buf ^ 1) * C::kBufBytes, regs[r]);
            __builtin_amdgcn_sched_barrier(0);
            const int kb = clampst(s + 1 + C::kDepth) * C::kKB;
            load_stage<C>(a_tile + kb * 34, w_tile + kb * 18, offs, regs[r]);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        }
    }

    if constexpr (!kIsums) {
        if constexpr (C::kWK > 1) {
            // add the other K-waves' partials to wave wk == 0's, in wave order;
            // the stage buffers are free after the loop's last barrier
            constexpr int kRegs = C::TM * C::TN * 16;
            float *red = reinterpret_cast<float *>(lds);
            if (wk > 0) {
                float *dst = red + ((wk - 1) * C::kWM * C::kWN + wmn) * kRegs * 64 + lane;
#pragma unroll
                for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
                        for (int r = 0; r < 16; ++r) dst[((tm * C::TN + tn) * 16 + r) * 64] = acc[tm][tn][r];
            }
            __syncthreads();
            if (wk > 0) return;
#pragma unroll
            for (int w2 = 1; w2 < C::kWK; ++w2) {
                const float *src = red + ((w2 - 1) * C::kWM * C::kWN + wmn) * kRegs * 64 + lane;
#pragma unroll
                for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[tm][tn][r] += src[((tm * C::TN + tn) * 16 + r) * 64];
            }
        }
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const int col = n0 + wave_n * C::TN * 32 + tn * 32 + li;
                if (col < n) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wave_m * C::TM * 32 + tm * 32 + mfma_row(lane, r);
                        if (row < m) store_through(&c[(size_t)row * n + col], acc[tm][tn][r] * 0.0625f);
                    }
                }
            }
    }
}

template <class C, bool kIsums>
hipError_t launch_q4_0(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n, int64_t k,
                       hipStream_t stream) {
    const dim3 grid((unsigned)(((n + C::kBN - 1) / C::kBN) * ((m + C::kBM - 1) / C::kBM)));
    hipLaunchKernelGGL((gemm_q4_0_kernel<C, kIsums>), grid, dim3(C::kThreads), C::kLdsBytes, stream,
                       static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, isums, (int)m, (int)n,
                       (int)(k / 32));
    return hipGetLastError();
}

// large problems: 128x128 tiles, 4 waves of 64x64, 4 blocks per stage
using Q40Big = Q40Config<128, 128, 2, 2, 4>;
// medium problems: 64x64 tiles, 4 waves of 32x32, 8 blocks per stage
using Q40Small = Q40Config<64, 64, 2, 2, 8>;
// medium problems with k % 256 != 0: 64x64 tiles, 2 waves of 64x32, 4 blocks per stage
using Q40Small4 = Q40Config<64, 64, 1, 2, 4>;
// small problems: 32x32 tiles, 2 waves each taking 4 of the stage's 8 blocks,
// loads two stages ahead (three was 5-10 % slower: fewer waves fit)
using Q40Tiny = Q40Config<32, 32, 1, 1, 8, 2, 2>;

// decode batches (at most one 32x32 tile per CU): 32x32 tiles, 8 waves each
// taking 4 of the stage's 32 blocks, loads two stages ahead
using Q40Mid = Q40Config<32, 32, 1, 1, 32, 8, 2>;

// between the two: 64x64 tiles, 4 waves of 32x32 twice over (2 K-waves each
// taking 8 of a 16-block stage), loads two stages ahead
using Q40SmallK2 = Q40Config<64, 64, 2, 2, 16, 2, 2>;

enum { kCfgBig = 0, kCfgSmall = 1, kCfgSmall4 = 2, kCfgTiny = 3, kCfgMid = 4, kCfgSmallK2 = 5, kCfgWhole = 6 };

int64_t tiles_of(int64_t m, int64_t n, int64_t bm, int64_t bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); }

}  // namespace

bool mfma_supported(int type, int64_t m, int64_t k) {
    (void)m;
    if (k > kMaxTiledK) return false;  // 32-bit load offsets
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return k % (32 * 4) == 0;  // Q40Small4 takes any k % 128 == 0
    // the super-block formats take any k % 256 == 0 (gemm_kquant.hip)
    return (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K || type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) && k % 256 == 0;
}

// Tile choice (measured on MI355X, 256 CUs): when the 32x32 tiles number at
// most one per CU (decode batches: m <= 64 at n = 4096), the 8-K-wave 32x32
// tile; else 128x128 tiles when there are at least two per CU, 64x64 tiles
// from 1.25 per CU, the 2-K-wave 64x64 tile from 0.75 per CU when K is long
// enough for its 16-block stages (256x4096x4096: 22.6 instead of 26.8 us), and
// the 2-K-wave 32x32 tile below that.
MfmaPlan plan_mfma(int type, int64_t m, int64_t n, int64_t k, int cus) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return plan_kquant(type, m, n, k, cus);
    MfmaPlan p;
    const int64_t enough = 2 * (int64_t)cus;
    if (k % (32 * Q40Mid::kKB) == 0 && tiles_of(m, n, 32, 32) <= cus) {
        p.config = kCfgMid;
    } else if (q4_0_small_supported(k) && 2 * tiles_of(m, n, 32, 96) >= cus && tiles_of(m, n, 32, 96) <= cus) {
        // whole-K 32x96 tiles, one per CU and one round (480x1536x1536:
        // 8.6 us against 9.8 us for the 2-K-wave 32x32 tile)
        p.config = kCfgWhole;
    } else if (tiles_of(m, n, 128, 128) >= enough) {
        p.config = kCfgBig;
    } else if (k % (32 * Q40Small::kKB) != 0) {
        p.config = kCfgSmall4;
    } else if (4 * tiles_of(m, n, 64, 64) >= 5 * (int64_t)cus) {
        p.config = kCfgSmall;
    } else if (k % (32 * Q40SmallK2::kKB) == 0 && k >= 2048 && 4 * tiles_of(m, n, 64, 64) >= 3 * (int64_t)cus) {
        p.config = kCfgSmallK2;
    } else {
        p.config = kCfgTiny;
    }
    return p;
}

hipError_t launch_mfma_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                               const MfmaPlan &plan, hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return launch_kquant_mul_mat(type, w, a, c, m, n, k, plan, stream);
    switch (plan.config) {
    case kCfgBig: return launch_q4_0<Q40Big, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgSmall: return launch_q4_0<Q40Small, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgTiny: return launch_q4_0<Q40Tiny, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgMid: return launch_q4_0<Q40Mid, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgSmallK2: return launch_q4_0<Q40SmallK2, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgWhole: return launch_q4_0_small(w, a, c, nullptr, m, n, k, stream);
    default: return launch_q4_0<Q40Small4, false>(w, a, c, nullptr, m, n, k, stream);
    }
}

hipError_t launch_mfma_block_isums(int type, const void *w, const void *a, int32_t *out, int64_t m, int64_t n,
                                   int64_t k, const MfmaPlan &plan, hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0)
        return launch_kquant_block_isums(type, w, a, out, m, n, k, plan, stream);
    switch (plan.config) {
    case kCfgBig: return launch_q4_0<Q40Big, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgSmall: return launch_q4_0<Q40Small, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgTiny: return launch_q4_0<Q40Tiny, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgMid: return launch_q4_0<Q40Mid, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgSmallK2: return launch_q4_0<Q40SmallK2, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgWhole: return launch_q4_0_small(w, a, nullptr, out, m, n, k, stream);
    default: return launch_q4_0<Q40Small4, true>(w, a, nullptr, out, m, n, k, stream);
    }
}

}  // namespace pfng
