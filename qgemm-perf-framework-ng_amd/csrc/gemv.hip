// q4_0 x q8_0 GEMV path (m <= 16, and up to 64 or 128 at k % 256 == 0) for gfx950: the
// weight stream is the roofline. Six kernels, picked in launch_gemv /
// launch_fused_gemv:
//
//   gemv_q4_0_m1_kernel        m == 1: one wavefront per weight row, one q4_0
//                              block pair (36 B) per lane, the activation row
//                              copied into LDS once per 16-row workgroup.
//   gemv_q4_0_pairs_kernel     m = 2..16 while the staged activations fit LDS:
//                              the same row/pair mapping, the m activation
//                              rows staged realigned with fp32 scales, a
//                              reduce-scatter across the wave at the end.
//   gemv_q4_0_kernel           m = 2..8 with longer rows (k % 256 == 0): groups
//                              of eight blocks (144 B, 16-byte aligned) per
//                              lane, L lanes per row, activations staged in
//                              LDS chunk by chunk (272 B per group: 8 x 32 int8
//                              bytes, then the 8 fp16 scales).
//   gemv_q4_0_fused_kernel     pfng_hip_compute for m <= 2: quantizes the fp32
//                              activation rows into LDS, then as the m1 kernel.
//   gemv_q4_0_mfma_chunk_kernel k % 256 == 0 from k = 512, from m = 3..6 (by
//                              k) up to m = 64 (k < 2048) or 128: 16x16 int8
//                              MFMA tiles of 16 weight rows, K split over the
//                              workgroup's 16 waves in 8-block groups (wave w
//                              takes groups w, w + 16, ..., one per round),
//                              each round's weights widened into registers
//                              once and the activation rows streamed through
//                              LDS in chunks of 16.
//
// Every lane issues all the loads of a step before any arithmetic, so the
// weight stream of the grid is in flight at once; weight rows are clamped so
// loads stay unconditional and only the stores are guarded.
//
// Arithmetic per block (exact integer part, then fp32):
//   w16 = 16 * (nibble - 8) packed as int8 (q4_0_unpack16), isum16 = sum w16 * a
//   (v_dot4_i32_i8), acc += float(isum16) * (dw * da); the output is acc / 16.
// |isum16| <= 16 * 32512 < 2^24, so float(isum16) is exact and the result equals
// the reference's dot (llama_reference.cpp:134-146) up to fp32 reassociation.
#include "device_common.h"
#include "kernels.h"

namespace pfng {

namespace {

constexpr int kGroupBlocks = 8;
constexpr int kGroupBytesLds = kGroupBlocks * 32 + 16;  // 272
constexpr int kChunkGroups = 16;                        // K chunk of 4096 elements per LDS fill
constexpr int kThreads = 256;

// Stage activation groups [g0, g0 + ng) of all m rows into LDS.
template <int M>
__device__ __forceinline__ void stage_q8_0_groups(const uint8_t *__restrict__ a, uint8_t *lds, int nb, int g0, int ng) {
    // one task per (row, block pair): 68 bytes, 4-byte aligned since nb is even
    const int pairs = ng * (kGroupBlocks / 2);
    for (int task = threadIdx.x; task < M * pairs; task += kThreads) {
        const int row = task / pairs;
        const int pr = task % pairs;
        const int blk = g0 * kGroupBlocks + pr * 2;
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a + ((size_t)row * nb + blk) * 34);
        uint32_t v[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) v[i] = src[i];
        uint32_t q0[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q0[i] = shift2(v[i], v[i + 1]);
        const int lg = pr / 4, lb = (pr % 4) * 2;  // group within chunk, first block within group
        uint8_t *gbase = lds + (row * kChunkGroups + lg) * kGroupBytesLds;
        uint4 *dq = reinterpret_cast<uint4 *>(gbase + lb * 32);
        dq[0] = make_uint4(q0[0], q0[1], q0[2], q0[3]);
        dq[1] = make_uint4(q0[4], q0[5], q0[6], q0[7]);
        dq[2] = make_uint4(v[9], v[10], v[11], v[12]);
        dq[3] = make_uint4(v[13], v[14], v[15], v[16]);
        *reinterpret_cast<uint32_t *>(gbase + 256 + lb * 2) = (v[0] & 0xffffu) | (v[8] & 0xffff0000u);
    }
}

// Nine 16-byte loads of eight consecutive q4_0 blocks (144 B, 16-byte aligned).
__device__ __forceinline__ void load_q4_0_group(const uint8_t *__restrict__ w, bool ok, size_t first_block,
                                                uint32_t (&wv)[36]) {
    if (ok) {
        const uint4 *src = reinterpret_cast<const uint4 *>(w + first_block * 18);
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            const uint4 t = src[i];
            wv[4 * i] = t.x;
            wv[4 * i + 1] = t.y;
            wv[4 * i + 2] = t.z;
            wv[4 * i + 3] = t.w;
        }
    } else {
        // decodes to zero weights
#pragma unroll
        for (int i = 0; i < 36; ++i) wv[i] = 0x88888888u;
    }
}

// isum16 of the first block of a q4_0 pair read at its natural two-byte
// offset, against the first block of a q8_0 pair likewise: weight dwords
// u[0..4] = d | qs[0..1], qs[2..5], ..., qs[14..15] | d', activation dwords
// v[0..8] = d | qs[0..1], qs[2..5], ..., qs[30..31] | d'. Both sit two bytes
// into their dwords, so byte b of u[k] (weight element 4k-2+b as its low
// nibble, 4k+14+b as its high nibble) faces activation element 4k-2+b in byte
// b of v[k] and element 4k+14+b in byte b of v[k+4]: no realignment, two more
// v_dot4, and the masks of u[0] and u[4] zero the bytes that hold scales.
__device__ __forceinline__ int q4_0_dot16_at2(const uint32_t *u, const uint32_t *v) {
    int s = __builtin_amdgcn_sdot4((int)q4_0_lo16<0xF0F00000u>(u[0]), (int)v[0], 0, false);
    s = __builtin_amdgcn_sdot4((int)q4_0_hi16<0xF0F00000u>(u[0]), (int)v[4], s, false);
#pragma unroll
    for (int k = 1; k < 4; ++k) {
        s = __builtin_amdgcn_sdot4((int)q4_0_lo16(u[k]), (int)v[k], s, false);
        s = __builtin_amdgcn_sdot4((int)q4_0_hi16(u[k]), (int)v[k + 4], s, false);
    }
    s = __builtin_amdgcn_sdot4((int)q4_0_lo16<0x0000F0F0u>(u[4]), (int)v[4], s, false);
    return __builtin_amdgcn_sdot4((int)q4_0_hi16<0x0000F0F0u>(u[4]), (int)v[8], s, false);
}

// acc + 16 * (dot of a q4_0 block pair with a q8_0 block pair): u = the pair's
// nine weight dwords as loaded, v = the activation pair's seventeen dwords.
// Per block acc = fma(float(isum16), dw * da, acc), the scale product exact.
__device__ __forceinline__ float q4_0_pair_dot16(const uint32_t (&u)[9], const uint32_t (&v)[17], float acc) {
    const int s0 = q4_0_dot16_at2(u, v);
    int s1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s1 = __builtin_amdgcn_sdot4((int)q4_0_lo16(u[5 + i]), (int)v[9 + i], s1, false);
        s1 = __builtin_amdgcn_sdot4((int)q4_0_hi16(u[5 + i]), (int)v[13 + i], s1, false);
    }
    acc = __builtin_fmaf((float)s0, fp16_product<false, false>(u[0], v[0]), acc);
    return __builtin_fmaf((float)s1, fp16_product<true, true>(u[4], v[8]), acc);
}

// Block j of a group sits at byte 18*j: fp16 d, then 16 bytes of nibbles.
template <int M>
__device__ __forceinline__ void gemv_q4_0_group(const uint32_t (&wv)[36], const uint8_t *gbase, float (&acc)[M]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t q[4], dw16;
        if (j % 2 == 0) {
            const int b = 9 * j / 2;
            dw16 = wv[b] & 0xffffu;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = shift2(wv[b + i], wv[b + i + 1]);
        } else {
            const int b = 9 * (j - 1) / 2;
            dw16 = wv[b + 4] >> 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = wv[b + 5 + i];
        }
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) q4_0_unpack16(q[i], lo[i], hi[i]);
        const float dw = fp16_to_f32(dw16);
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            const uint8_t *ab = gbase + mi * kChunkGroups * kGroupBytesLds;
            const uint4 a0 = *reinterpret_cast<const uint4 *>(ab + j * 32);
            const uint4 a1 = *reinterpret_cast<const uint4 *>(ab + j * 32 + 16);
            const float da = fp16_to_f32(*reinterpret_cast<const uint16_t *>(ab + 256 + 2 * j));
            int s = __builtin_amdgcn_sdot4((int)lo[0], (int)a0.x, 0, false);
            s = __builtin_amdgcn_sdot4((int)lo[1], (int)a0.y, s, false);
            s = __builtin_amdgcn_sdot4((int)lo[2], (int)a0.z, s, false);
            s = __builtin_amdgcn_sdot4((int)lo[3], (int)a0.w, s, false);
            s = __builtin_amdgcn_sdot4((int)hi[0], (int)a1.x, s, false);
            s = __builtin_amdgcn_sdot4((int)hi[1], (int)a1.y, s, false);
            s = __builtin_amdgcn_sdot4((int)hi[2], (int)a1.z, s, false);
            s = __builtin_amdgcn_sdot4((int)hi[3], (int)a1.w, s, false);
            acc[mi] = fmaf((float)s, dw * da, acc[mi]);
        }
    }
}

template <int M>
__global__ __launch_bounds__(kThreads) void gemv_q4_0_kernel(const uint8_t *__restrict__ w,
                                                            const uint8_t *__restrict__ a, float *__restrict__ c,
                                                            int n, int nb, int lanes_per_row) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int L = lanes_per_row;
    const int rows_per_wave = 64 / L;
    const int slot = lane / L;
    const int sl = lane % L;
    const int row = (blockIdx.x * (kThreads / 64) + wave) * rows_per_wave + slot;
    const bool row_ok = row < n;
    const int groups = nb / kGroupBlocks;

    float acc[M];
#pragma unroll
    for (int i = 0; i < M; ++i) acc[i] = 0.0f;

    for (int g0 = 0; g0 < groups; g0 += kChunkGroups) {
        const int ng = groups - g0 < kChunkGroups ? groups - g0 : kChunkGroups;
        // issue this lane's first weight group before staging, so that the HBM
        // latency overlaps the activation staging and the barrier
        int lg = sl;
        uint32_t wv[36];
        load_q4_0_group(w, row_ok && lg < ng, (size_t)row * nb + (size_t)(g0 + lg) * kGroupBlocks, wv);
        if (g0) __syncthreads();
        stage_q8_0_groups<M>(a, lds, nb, g0, ng);
        __syncthreads();
        while (lg < ng) {
            uint32_t cur[36];
#pragma unroll
            for (int i = 0; i < 36; ++i) cur[i] = wv[i];
            const int next = lg + L;
            if (next < ng) load_q4_0_group(w, row_ok, (size_t)row * nb + (size_t)(g0 + next) * kGroupBlocks, wv);
            gemv_q4_0_group<M>(cur, lds + lg * kGroupBytesLds, acc);
            lg = next;
        }
    }
    // reduce the L lanes of each row slot
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
        float v = acc[mi];
        for (int o = L / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        acc[mi] = v;
    }
    // after the butterfly every lane of the slot holds all M sums; lane sl
    // stores activation rows sl, sl + L, ... (L may be smaller than M)
    if (row_ok) {
#pragma unroll
        for (int mi = 0; mi < M; ++mi)
            if (mi % L == sl) c[(size_t)mi * n + row] = acc[mi] * 0.0625f;
    }
}

// m == 1. Each lane owns one q4_0 block pair of its row (36 bytes, nine dword
// loads, 4-byte aligned when k % 64 == 0) and reads the matching q8_0 block
// pair of the activation row (68 bytes, seventeen dwords); both pairs are
// dotted as loaded (q4_0_pair_dot16: the first blocks at their common
// two-byte offset, nothing realigned). All of a lane's loads are issued
// before any arithmetic, so each lane pays one memory round trip. One
// wavefront covers 64 block pairs of one row (a whole row at k = 4096).
//
// kLdsAct (activation rows up to 64 KB): workgroups of 16 rows copy the
// activation row into LDS once, and the 16 waves read it from there instead
// of each fetching it from L2. The copy uses direct loads into LDS
// (global_load_lds_dwordx4: lane i of a wave writes 16 bytes at the wave's
// LDS base + 16 i, no VGPR round trip), and every lane issues the three load
// instructions of its first weight pair (clamped into the row, so they are
// always issued) before any wave waits: each wave then waits for its own
// copies only (s_waitcnt vmcnt(3): memory loads complete in issue order, so
// at most the three weight loads are left) and meets the others at the
// barrier, and the activation's trip from L2 overlaps the weight stream
// instead of preceding it. Without kLdsAct, 4-row workgroups read the
// activation directly.
template <bool kLdsAct>
__global__ __launch_bounds__(kLdsAct ? 1024 : kThreads) void gemv_q4_0_m1_kernel(const uint8_t *__restrict__ w,
                                                                               const uint8_t *__restrict__ a,
                                                                               float *__restrict__ c, int n, int nb) {
    constexpr int kBlockThreads = kLdsAct ? 1024 : kThreads;
    extern __shared__ __align__(16) uint8_t sact[];
    const int lane = threadIdx.x & 63;
    // the row is uniform across the wave: its base address lives in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = blockIdx.x * (kBlockThreads / 64) + wave;
    const int lrow = row < n ? row : n - 1;  // clamped: loads stay unconditional, the store is guarded
    const uint8_t *wrow = w + (size_t)lrow * nb * 18;
    const int np = nb / 2;
    const uint8_t *act = a;
    float acc = 0.0f;
    int p = lane;
    if constexpr (kLdsAct) {
        // 16-byte chunks (the row base is 16-byte aligned), wave w taking
        // chunks 64 w + lane (+ 1024 per round), then the dword tail (nb is
        // even, so the row is a whole number of dwords) from the last wave
        const int n16 = nb * 34 / 16, nd = nb * 34 / 4;
        for (int c0 = wave * 64; c0 < n16; c0 += kBlockThreads) {
            if (c0 + lane < n16)
                __builtin_amdgcn_global_load_lds(a + (size_t)(c0 + lane) * 16, (__attribute__((address_space(3))) void *)(sact + c0 * 16),
                                                 16, 0, 0);
        }
        if (wave == kBlockThreads / 64 - 1 && 4 * n16 + lane < nd)
            __builtin_amdgcn_global_load_lds(a + (size_t)(4 * n16 + lane) * 4, (__attribute__((address_space(3))) void *)(sact + n16 * 16),
                                             4, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        const int pc = lane < np ? lane : np - 1;
        const uint32_t *ws = reinterpret_cast<const uint32_t *>(wrow + (uint32_t)pc * 36u);
        uint32_t u[9], v[17];
#pragma unroll
        for (int i = 0; i < 9; ++i) u[i] = ws[i];
        asm volatile("s_waitcnt vmcnt(3)\n\ts_barrier" ::: "memory");
        const uint32_t *as = reinterpret_cast<const uint32_t *>(sact + (size_t)pc * 68);
#pragma unroll
        for (int i = 0; i < 17; ++i) v[i] = as[i];
        // lanes past the row's last pair dot a clamped duplicate and drop it
        // (a select, not a branch, so the loads stay ahead of the wait)
        const float first = q4_0_pair_dot16(u, v, 0.0f);
        acc = lane < np ? first : 0.0f;
        p += 64;
        act = sact;
    }
    for (; p < np; p += 64) {
        const uint32_t *ws = reinterpret_cast<const uint32_t *>(wrow + (uint32_t)p * 36u);
        const uint32_t *as = reinterpret_cast<const uint32_t *>(act + (size_t)p * 68);
        uint32_t u[9], v[17];
#pragma unroll
        for (int i = 0; i < 9; ++i) u[i] = ws[i];
#pragma unroll
        for (int i = 0; i < 17; ++i) v[i] = as[i];
        __builtin_amdgcn_sched_barrier(0);
        acc = q4_0_pair_dot16(u, v, acc);
    }
    acc = wave_sum_lane63(acc);
    if (row < n && lane == 63) c[row] = acc * 0.0625f;
}

// m = 2..16 when the m activation rows fit the 160 KB of LDS in the layout below.
// Workgroups of 16 weight rows stage the activations once: each q8_0 block
// pair of each row becomes 64 realigned int8 bytes (17-dword stride, so lanes
// reading consecutive pairs hit distinct banks) plus its two scales widened to
// fp32 in a separate array. Each wavefront then takes one weight row: lane p
// owns block pair p (nine weight dwords, as gemv_q4_0_m1_kernel), decodes it
// once and dots it with the m activation pairs read from LDS, so the inner
// loop is the v_dot4 work and the fp32 scaling only. One wave covers a
// 4096-wide K stretch per step.
//
// Cross-lane reduction: P = the largest power of two <= m rows go through a
// reduce-scatter butterfly in which every exchange halves the values a lane
// carries (log2(P) exchanges of P-1 values in all, then a plain butterfly over
// the lane bits left), the other m - P rows through a plain butterfly each.
// Lane l's accumulator j (j < P) holds activation row j ^ f(l), f(l) being the
// lane bits the exchanges run over, so that every lane keeps the lower half
// and sends the upper half: the lane dependence sits in the LDS read address
// and accumulators are only ever indexed by constants (a lane-dependent
// choice between accumulators becomes a scratch-memory array). For some m, P
// is the next power of two instead: accumulators of rows >= m then read a
// clamped row, only ever combine with each other, and are never stored.
constexpr int kPairsThreads = 1024;
constexpr int kPairDwords = 17;  // 16 int8 dwords + 1 pad

// int8 part, rounded up to 16 bytes, then the fp32 scale pairs; the size
// allows for the rounding: m * (nb / 2) * 76 + 16 bytes
__host__ __device__ constexpr int64_t pairs_scale_offset(int64_t m, int64_t nb) {
    return (m * (nb / 2) * kPairDwords * 4 + 15) / 16 * 16;
}
__host__ __device__ constexpr int64_t pairs_lds_bytes(int64_t m, int64_t nb) {
    return m * (nb / 2) * (kPairDwords * 4 + 8) + 16;
}

constexpr int kPairsMaxM = 16;
constexpr int64_t kPairsMaxLds = 160 * 1024;  // one workgroup per CU holds the whole LDS

template <int M>
__global__ __launch_bounds__(kPairsThreads) void gemv_q4_0_pairs_kernel(const uint8_t *__restrict__ w,
                                                                       const uint8_t *__restrict__ a,
                                                                       float *__restrict__ c, int n, int nb) {
    // reduce-scatter width: rows beyond the largest power of two <= M cost a
    // plain butterfly each; at M = 7 and M >= 13 padding to the next power of
    // two (dummy rows, never stored) measured faster
    constexpr int P = M == 7 || M >= 13 ? pow2_ceil16(M) : pow2_floor16(M);
    constexpr int NA = P > M ? P : M;              // accumulators per lane
    constexpr int kLaneShift = 6 - log2_pow2(P);  // lanes per reduce-scatter result: 1 << kLaneShift
    extern __shared__ __align__(16) uint8_t lds[];
    const int np = nb / 2;
    uint32_t *xq = reinterpret_cast<uint32_t *>(lds);                          // [M][np][17]
    float2 *xd = reinterpret_cast<float2 *>(lds + pairs_scale_offset(M, nb));  // [M][np]
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kPairsThreads / 64) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lrow = row < n ? row : n - 1;  // clamped: loads stay unconditional, the store is guarded
    const uint8_t *wrow = w + (size_t)lrow * nb * 18;
    const int ntask = M * np;
    // task = row * np + pair: the pair's 68 bytes (4-byte aligned, nb even)
    // realigned into xq, its scales widened into xd
    auto stage = [&](const uint32_t (&v)[17], int task, bool store) {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = shift2(v[i], v[i + 1]);
        const float2 d = make_float2(fp16_to_f32(v[0] & 0xffffu), fp16_to_f32(v[8] >> 16));
        if (store) {
            uint32_t *dst = xq + (size_t)task * kPairDwords;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                dst[i] = q[i];
                dst[8 + i] = v[9 + i];
            }
            xd[task] = d;
        }
    };
    // each thread's first staging task (the only one while m * k / 64 <=
    // 1024, so always at k <= 4096), then the lane's first weight pair
    // (clamped into the row, so always issued): the staging waits for its
    // own loads only, and the weights' trip from HBM overlaps it and the
    // barrier. Threads without a task load nothing (clamping them onto the
    // last task would send every idle wave of the grid to one L2 channel).
    int task = threadIdx.x;
    uint32_t v0[17];
    if (task < ntask) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a + (size_t)task * 68);
#pragma unroll
        for (int i = 0; i < 17; ++i) v0[i] = src[i];
    } else {
#pragma unroll
        for (int i = 0; i < 17; ++i) v0[i] = 0;
    }
    __builtin_amdgcn_sched_barrier(0);
    const int pc = lane < np ? lane : np - 1;
    uint32_t u0[9];
    {
        const uint32_t *ws = reinterpret_cast<const uint32_t *>(wrow + (uint32_t)pc * 36u);
#pragma unroll
        for (int i = 0; i < 9; ++i) u0[i] = ws[i];
    }
    __builtin_amdgcn_sched_barrier(0);
    use_here(v0);
    stage(v0, task, task < ntask);
    for (task += kPairsThreads; task < ntask; task += kPairsThreads) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a + (size_t)task * 68);
        uint32_t v[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) v[i] = src[i];
        stage(v, task, true);
    }
    __syncthreads();
    redefine_here(u0);  // the weights are decoded after the barrier, which then waits for the staging only
    const int f = lane >> kLaneShift;  // < P
    int arow[NA];                      // activation row read for accumulator j (clamped)
#pragma unroll
    for (int j = 0; j < NA; ++j) {
        const int r = j < P ? j ^ f : j;
        arow[j] = r < M ? r : M - 1;
    }
    // acc[j] += the pair's two block dots with activation row arow[j]
    auto pair_step = [&](const uint32_t (&u)[9], int p, float (&acc)[NA]) {
        // block 2p: d at byte 0, qs at 2 (realign by two bytes); block 2p+1: d at 18, qs at 20
        uint32_t lo0[4], hi0[4], lo1[4], hi1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q4_0_unpack16(shift2(u[i], u[i + 1]), lo0[i], hi0[i]);
            q4_0_unpack16(u[5 + i], lo1[i], hi1[i]);
        }
        const float dw0 = fp16_to_f32(u[0] & 0xffffu), dw1 = fp16_to_f32(u[4] >> 16);
#pragma unroll
        for (int j = 0; j < NA; ++j) {
            const int t = arow[j] * np + p;
            const uint32_t *x = xq + (size_t)t * kPairDwords;
            const float2 da = xd[t];
            int s0 = 0, s1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s0 = __builtin_amdgcn_sdot4((int)lo0[i], (int)x[i], s0, false);
                s1 = __builtin_amdgcn_sdot4((int)lo1[i], (int)x[8 + i], s1, false);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s0 = __builtin_amdgcn_sdot4((int)hi0[i], (int)x[4 + i], s0, false);
                s1 = __builtin_amdgcn_sdot4((int)hi1[i], (int)x[12 + i], s1, false);
            }
            acc[j] += (float)s0 * (dw0 * da.x);
            acc[j] += (float)s1 * (dw1 * da.y);
        }
    };
    float acc[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) acc[j] = 0.0f;
    pair_step(u0, pc, acc);
#pragma unroll
    for (int j = 0; j < NA; ++j) acc[j] = lane < np ? acc[j] : 0.0f;  // past the last pair: a clamped duplicate
    for (int p = lane + 64; p < np; p += 64) {
        const uint32_t *ws = reinterpret_cast<const uint32_t *>(wrow + (uint32_t)p * 36u);
        uint32_t u[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) u[i] = ws[i];
        __builtin_amdgcn_sched_barrier(0);
        pair_step(u, p, acc);
    }
    // reduce-scatter over accumulators 0..P-1 (exchange offsets 32, 16, ...),
    // then a DPP sum over the 64 / P lanes left: the group's last lane holds it
    constexpr int G = 1 << kLaneShift;
    reduce_scatter_steps<P / 2, 32>(acc);
    acc[0] = group_sum_dpp<G>(acc[0]);
#pragma unroll
    for (int j = P; j < M; ++j) acc[j] = wave_sum_lane63(acc[j]);
    if (row < n) {
        if ((lane & (G - 1)) == G - 1 && f < M) c[(size_t)f * n + row] = acc[0] * 0.0625f;
        if (lane == 63) {
#pragma unroll
            for (int j = P; j < M; ++j) c[(size_t)j * n + row] = acc[j] * 0.0625f;
        }
    }
}

// k % 256 == 0 from k = 512 (16 waves of 8 blocks per round; round r takes
// blocks 8 (16 r + wave) .. + 8 of every row while they exist, so waves can run
// different numbers of rounds, or none below k = 4096, the partial sums
// staying in registers) from m = q4_0_tiles_min_m(k): 16x16 int8 MFMA tiles
// over C = ceil(m / 16) chunks of 16 activation rows (m up to
// gemv_tiles_max_m(k)). A workgroup takes 16 weight rows (output columns).
// Per block lane l takes weight row l % 16 (B) and activation row l % 16 of
// the chunk (A) with K positions 4q..4q+3 and 16+4q..16+4q+3, q = l / 16: one
// nibble dword gives both (low nibbles, then high), and the activation's two
// dwords sit at the same byte offsets; the first block of a pair sits two
// bytes into its dwords (realigned with v_alignbyte), the second is
// dword-aligned. One v_mfma_i32_16x16x32_i8 per block gives 16 S_b.
constexpr int kMf8Blocks = 8;  // blocks per wave
constexpr int kMf8Waves = 16;

// Each wave copies its 8-block slice of the 16 weight rows
// once (144 bytes a row) and widens it once into registers (the nibbles as
// 16 (q - 8) int8 operands, the fp16 scales); chunk c's activation slice
// (272 bytes a row) arrives in two halves, H0 = slice bytes 0..143 (blocks
// 0..3) and H1 = bytes 128..271 (blocks 4..7), each into its own LDS buffer,
// refilled with chunk c + 1 as soon as the wave has read it (the copy of
// H0(c + 1) runs while H1(c) is multiplied, H1(c + 1)'s while H0(c + 1) is).
// Every wait is for the instructions that wrote one buffer (loads complete in
// issue order). Activation rows past m repeat row m - 1 (not stored). Per
// block the scale product dw * da comes from the matrix core (one-hot
// v_mfma_f32_16x16x16_f16), then acc += float(16 S_b) * P per result.
// Measured at 4096 x 4096 against the former kernel that copied each chunk's
// weight and activation slice together in two halves (us): q4_0 m = 6 5.33 /
// 5.15, m = 8 5.42 / 5.16, m = 16 5.83 / 5.28; below m = 6 the pairs kernel
// is faster (m = 5 4.93 / 5.15).
constexpr int kQ40ChunkWaveBytes = 9 * 1024;  // weight run, H0, H1: 3 KB each
// A wave stores its partials as soon as it is done and one barrier suffices
// (against a first barrier and shared buffers, 4096 x 4096): with one chunk
// (m <= 16) into a 16 KB region of their own past the wave buffers (m = 16
// 5.06 -> 5.01 us, m = 8 4.75 -> 4.72), with more chunks into the wave's own
// buffers (C KB of its 9), which no other wave reads and whose last copy has
// landed once it is done (m = 32 6.88 -> 6.77 us, m = 128 15.32 -> 15.20).
template <int C> constexpr int q4_0_chunk_lds_bytes() {
    return kMf8Waves * kQ40ChunkWaveBytes + (C == 1 ? kMf8Waves * 1024 : 0);
}

template <int C, int kG>
__global__ __launch_bounds__(kMf8Waves * 64) void gemv_q4_0_mfma_chunk_kernel(const uint8_t *__restrict__ w,
                                                                              const uint8_t *__restrict__ a,
                                                                              float *__restrict__ c, int m, int n,
                                                                              int groups) {
    static_assert(C >= 1 && C <= kMaxGemvChunks, "at most kMaxGemvChunks chunks of 16 activation rows");
    // 256-element groups of a row (k == 256 ng, ng >= 2): kG when it is fixed at
    // compile time (k = 4096: one round, constant strides), else groups
    const int ng = kG > 0 ? kG : groups;
    const int nb = kMf8Blocks * ng;
    const uint32_t kARow = (uint32_t)nb * 34;
    constexpr int kH = run_copies<16, 9>();
    static_assert(kH * 1024 <= 3072, "3 KB per run");
    static_assert(4 * C * 64 * 4 <= kQ40ChunkWaveBytes, "a wave's partials fit its buffers");
    static_assert(q4_0_chunk_lds_bytes<C>() <= 160 * 1024, "the LDS of one CU");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int n0 = blockIdx.x * 16;
    uint8_t *wl = lds + wave * kQ40ChunkWaveBytes, *h0 = wl + 3072, *h1 = wl + 6144;
    float acc[C][4];
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[ch][r] = 0.0f;
    // round rnd takes the wave's K slice 16 rnd + wave of every row; the next
    // round's copies start once the last round's buffers have been read
    // this wave's rounds: its 8-block groups wave, wave + 16, ... below ng
    const int my_rounds = (ng - wave + kMf8Waves - 1) / kMf8Waves;
#pragma clang loop unroll(disable)
    for (int rnd = 0; rnd < my_rounds; ++rnd) {
        // a lane index the compiler cannot carry across rounds: the per-lane
        // copy offsets and LDS addresses are recomputed per round instead of
        // held in registers for the whole loop (one round with kG: no need)
        int cl = lane;
        if constexpr (kG == 0) asm volatile("" : "+v"(cl));
        const int li = cl & 15, q = cl >> 4;
        // the last round's LDS reads are done before its buffers are refilled (in
        // round 0 there is nothing to wait for; a wait in the later rounds only
        // would make the compiler peel round 0)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int kb0 = (kMf8Waves * rnd + wave) * kMf8Blocks;  // the wave's first block
        const uint8_t *asrc = a + kb0 * 34;  // the wave's slice of activation row 0
        auto copy_h0 = [&](int ch) { copy_run<C, 16, 9>(asrc + (size_t)ch * 16 * kARow, kARow, 0, m - 16 * ch, h0, cl); };
        auto copy_h1 = [&](int ch) { copy_run<C, 16, 9>(asrc + (size_t)ch * 16 * kARow, kARow, 8, m - 16 * ch, h1, cl); };
        copy_run<C, 16, 9>(w + ((size_t)n0 * nb + kb0) * 18, nb * 18, 0, n - n0, wl, cl);
        copy_h0(0);
        copy_h1(0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // weights and H0(0)
        // the weight slice, once: block j's 8 int8 operands of this lane and its scale
        const uint8_t *wr = wl + li * 144;
        uint64_t bop[kMf8Blocks];
        uint32_t dw[kMf8Blocks];
    #pragma unroll
        for (int j = 0; j < kMf8Blocks; ++j) {
            uint32_t wq;
            if ((j & 1) == 0) {  // two bytes into its dwords
                const uint32_t *w0 = reinterpret_cast<const uint32_t *>(wr + j * 18 + 4 * q);
                wq = shift2(w0[0], w0[1]);
            } else {
                wq = *reinterpret_cast<const uint32_t *>(wr + j * 18 + 2 + 4 * q);
            }
            bop[j] = (uint64_t)q4_0_lo16(wq) | ((uint64_t)q4_0_hi16(wq) << 32);
            const uint32_t dw_all = *reinterpret_cast<const uint16_t *>(wr + j * 18);  // every lane reads: no branch
            dw[j] = q == 0 ? dw_all : 0u;
        }
    #pragma unroll
        for (int ch = 0; ch < C; ++ch) {
            // block j of the chunk row li: slice byte 34 j, in H0 (j < 4) or H1 (from slice byte 128)
            auto block = [&](int j) {
                const uint8_t *ar = (j < 4 ? h0 + li * 144 : h1 + li * 144 - 128) + j * 34;
                uint32_t x0, x1;
                if ((j & 1) == 0) {
                    const uint32_t *a0 = reinterpret_cast<const uint32_t *>(ar + 4 * q);
                    x0 = shift2(a0[0], a0[1]);
                    x1 = shift2(a0[4], a0[5]);
                } else {
                    const uint32_t *a1 = reinterpret_cast<const uint32_t *>(ar + 2 + 4 * q);
                    x0 = a1[0];
                    x1 = a1[4];
                }
                const i32x4 s16 = mfma_i8_16x16x32((uint64_t)x0 | ((uint64_t)x1 << 32), bop[j], (i32x4){0, 0, 0, 0});
                const uint32_t da_all = *reinterpret_cast<const uint16_t *>(ar);  // every lane reads: no branch
                const uint32_t da = q == 0 ? da_all : 0u;
                const f16x4 pa = __builtin_bit_cast(f16x4, make_uint2(da, 0u));
                const f16x4 pb = __builtin_bit_cast(f16x4, make_uint2(dw[j], 0u));
                const f32x4 p = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, pb, (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    #pragma unroll
                for (int r = 0; r < 4; ++r) acc[ch][r] = __builtin_fmaf((float)s16[r], p[r], acc[ch][r]);
            };
            if (ch > 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // H0(ch)
    #pragma unroll
            for (int j = 0; j < 4; ++j) block(j);
            if (ch + 1 < C) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // H0 read: refill it
                copy_h0(ch + 1);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // H1(ch)
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
    #pragma unroll
            for (int j = 4; j < kMf8Blocks; ++j) block(j);
            if (ch + 1 < C) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // H1 read: refill it
                copy_h1(ch + 1);
            }
        }
    }
    // wave partials through LDS, each wave's in a region only it writes
    // ([group g = 4 chunk + r][lane]); wave w adds groups w, w + 16, ... over
    // the waves in wave order and stores them
    const int li = lane & 15, q = lane >> 4;
    // wave v's partials at red + v * kStride: a compile-time stride, so the
    // reads below take immediate offsets from one address
    float *red = reinterpret_cast<float *>(lds + (C == 1 ? kMf8Waves * kQ40ChunkWaveBytes : 0));
    constexpr int kStride = (C == 1 ? 1024 : kQ40ChunkWaveBytes) / 4;
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * kStride + (ch * 4 + r) * 64 + lane] = acc[ch][r];
    __syncthreads();
    const int col = n0 + li;
    for (int g = wave; g < 4 * C; g += kMf8Waves) {
        float s = red[g * 64 + lane];
        for (int v = 1; v < kMf8Waves; ++v) s += red[v * kStride + g * 64 + lane];
        const int row = 16 * (g / 4) + 4 * q + g % 4;
        if (col < n && row < m) store_through(&c[(size_t)row * n + col], s * 0.0625f);
    }
}

// One launch of gemv_q4_0_mfma_chunk_kernel with C chunks over ng 256-element
// groups, the k = 4096 form (16 groups, one round) where it applies.
template <int C>
void launch_q4_0_chunk(const uint8_t *w, const uint8_t *a, float *c, int m, int n, int ng, hipStream_t stream) {
    const dim3 grid((unsigned)((n + 15) / 16)), block(kMf8Waves * 64);
    const size_t lds = (size_t)q4_0_chunk_lds_bytes<C>();
    if (ng == kMf8Waves)
        hipLaunchKernelGGL((gemv_q4_0_mfma_chunk_kernel<C, kMf8Waves>), grid, block, lds, stream, w, a, c, m, n, ng);
    else
        hipLaunchKernelGGL((gemv_q4_0_mfma_chunk_kernel<C, 0>), grid, block, lds, stream, w, a, c, m, n, ng);
}

// Fused activation quantization + GEMV (m <= 2): each workgroup quantizes the
// m fp32 activation rows into q8_0 blocks in LDS (the same arithmetic as
// quantize_q8_0_kernel, so the bytes equal the standalone quantizer's), then
// its 16 waves each take one weight row as gemv_q4_0_m1_kernel does, reading
// the activation pairs from LDS. This saves the quantizer's launch and its
// round trip through HBM; the quantization is repeated per workgroup but costs
// m * k / 1024 elements per thread.
constexpr int kFusedThreads = 1024;

template <int M>
__global__ __launch_bounds__(kFusedThreads) void gemv_q4_0_fused_kernel(const uint8_t *__restrict__ w,
                                                                       const float *__restrict__ x,
                                                                       float *__restrict__ c, int n, int nb) {
    extern __shared__ __align__(16) uint8_t aq[];  // M rows of nb q8_0 blocks, HBM layout
    const int tid = threadIdx.x, sub = tid & 7, lane = tid & 63;
    const int row = blockIdx.x * (kFusedThreads / 64) + __builtin_amdgcn_readfirstlane((int)(tid >> 6));
    const int lrow = row < n ? row : n - 1;
    const uint8_t *wrow = w + (size_t)lrow * nb * 18;
    const int np = nb / 2, nblk = M * nb;
    // one quantization task = 4 elements of one block (8 lanes per block)
    auto quantize = [&](const float4 &v, int blk, bool store) {
        float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        amax = group_max<8>(amax);
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint32_t q = q8_quantize4(v, id);
        if (store) {
            uint16_t *ob = reinterpret_cast<uint16_t *>(aq + blk * 34);
            ob[1 + 2 * sub] = (uint16_t)(q & 0xffffu);
            ob[2 + 2 * sub] = (uint16_t)(q >> 16);
            if (sub == 0) ob[0] = (uint16_t)f32_to_fp16_bits(d);
        }
    };
    // the activations of each thread's first M tasks (all of them while
    // k <= 4096), then the first weight pair (all clamped, so the loads are
    // unconditional): the quantization waits for its own loads only, and the
    // weights' trip from HBM overlaps it and the barrier
    constexpr int kTaskStride = kFusedThreads / 8;
    int blk = tid >> 3;
    float4 x0[M];
#pragma unroll
    for (int t = 0; t < M; ++t) {
        const int b = blk + t * kTaskStride;
        x0[t] = *reinterpret_cast<const float4 *>(x + (size_t)(b < nblk ? b : nblk - 1) * 32 + sub * 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int pc = lane < np ? lane : np - 1;
    uint32_t u0[9];
    {
        const uint32_t *ws = reinterpret_cast<const uint32_t *>(wrow + (uint32_t)pc * 36u);
#pragma unroll
        for (int i = 0; i < 9; ++i) u0[i] = ws[i];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < M; ++t) quantize(x0[t], blk + t * kTaskStride, blk + t * kTaskStride < nblk);
    for (blk += M * kTaskStride; blk < nblk; blk += kTaskStride)
        quantize(*reinterpret_cast<const float4 *>(x + (size_t)blk * 32 + sub * 4), blk, true);
    __syncthreads();
    float acc[M];
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
        const uint32_t *as = reinterpret_cast<const uint32_t *>(aq + (mi * nb + 2 * pc) * 34);
        uint32_t v[17];
#pragma unroll
        for (int i = 0; i < 17; ++i) v[i] = as[i];
        const float first = q4_0_pair_dot16(u0, v, 0.0f);
        acc[mi] = lane < np ? first : 0.0f;  // lanes past the last pair drop their clamped duplicate
    }
    for (int p = lane + 64; p < np; p += 64) {
        const uint32_t *ws = reinterpret_cast<const uint32_t *>(wrow + (uint32_t)p * 36u);
        uint32_t u[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) u[i] = ws[i];
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            const uint32_t *as = reinterpret_cast<const uint32_t *>(aq + (mi * nb + 2 * p) * 34);
            uint32_t v[17];
#pragma unroll
            for (int i = 0; i < 17; ++i) v[i] = as[i];
            acc[mi] = q4_0_pair_dot16(u, v, acc[mi]);
        }
    }
    // the same sums as the unfused kernels, so the outputs are equal bit for
    // bit: m == 1 as gemv_q4_0_m1_kernel, m == 2 as gemv_q4_0_pairs_kernel<2>
    // (one exchange between the wave halves, then a 32-lane DPP sum)
    static_assert(M == 1 || M == 2, "fused for m <= 2");
    if constexpr (M == 1) {
        const float v = wave_sum_lane63(acc[0]);
        if (row < n && lane == 63) c[row] = v * 0.0625f;
    } else {
        const bool up = lane >= 32;
        float x = up ? acc[1] : acc[0];
        const float y = up ? acc[0] : acc[1];
        x += xor_shfl<32>(y);
        x = group_sum_dpp<32>(x);
        if (row < n && (lane & 31) == 31) c[(size_t)(up ? 1 : 0) * n + row] = x * 0.0625f;
    }
}

template <int M>
hipError_t launch_fused_m(const void *w, const float *x, float *c, int64_t n, int64_t k, hipStream_t stream) {
    const int nb = (int)(k / 32);
    const dim3 grid((unsigned)((n + kFusedThreads / 64 - 1) / (kFusedThreads / 64)));
    hipLaunchKernelGGL(gemv_q4_0_fused_kernel<M>, grid, dim3(kFusedThreads), (size_t)M * nb * 34, stream,
                       static_cast<const uint8_t *>(w), x, c, (int)n, nb);
    return hipGetLastError();
}

// k the chunked MFMA tile kernel takes: groups of 8 blocks (256 elements; the
// slices and rows stay 16-byte aligned at every k % 256), from k = 512 (below
// 4096 the waves past the last group idle)
bool q4_0_tiles_take_k(int64_t k) { return k % 256 == 0 && k >= 512; }

// Smallest m from which the tile kernel runs, measured at n = 4096 against the
// pairs and group kernels (us, tile / other): k = 512 m = 3 2.97 / 3.34;
// k = 1024 m = 3 3.30 / 3.41; k = 2048 m = 4 3.90 / 4.06 (m = 3 3.89 / 3.57);
// k = 3072 m = 5 4.33 / 4.63 (m = 4 4.37 / 4.22); k = 4096 m = 6 5.15 / 5.33
// (m = 5 5.15 / 4.93); above 4096 m = 5 (k = 8192 7.91 / 8.13-8.58, k = 12288
// 10.65 / 11.07-11.76, k = 11008 9.65 / 13.07).
int q4_0_tiles_min_m(int64_t k) {
    if (k <= 1024) return 3;
    if (k <= 2048) return 4;
    return k == 4096 ? 6 : 5;
}

template <int M>
hipError_t launch_gemv_q4_0_m(const void *w, const void *a, float *c, int64_t n, int64_t k, hipStream_t stream) {
    const int nb = (int)(k / 32);
    if (M >= q4_0_tiles_min_m(k) && q4_0_tiles_take_k(k)) {  // gemv_q4_0_mfma_chunk_kernel, one chunk
        launch_q4_0_chunk<1>(static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, M, (int)n,
                             (int)(k / 256), stream);
        return hipGetLastError();
    }
    if (k % 64 == 0 && pairs_lds_bytes(M, nb) <= kPairsMaxLds) {
        const int grid = (int)((n + kPairsThreads / 64 - 1) / (kPairsThreads / 64));
        hipLaunchKernelGGL(gemv_q4_0_pairs_kernel<M>, dim3(grid), dim3(kPairsThreads), (size_t)pairs_lds_bytes(M, nb),
                           stream, static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, (int)n, nb);
        return hipGetLastError();
    }
    if constexpr (M <= 8) {
        // longer rows: groups of 8 blocks per lane, activation chunks in LDS (k % 256 == 0)
        const int groups = nb / kGroupBlocks;
        const int gcap = groups < kChunkGroups ? groups : kChunkGroups;
        int L = 1;
        while (L * 2 <= gcap) L *= 2;
        const int rows_per_block = (kThreads / 64) * (64 / L);
        const int grid = (int)((n + rows_per_block - 1) / rows_per_block);
        const size_t lds = (size_t)M * kChunkGroups * kGroupBytesLds;
        hipLaunchKernelGGL(gemv_q4_0_kernel<M>, dim3(grid), dim3(kThreads), lds, stream,
                           static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, (int)n, nb, L);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Fusing pays only while the quantization repeated in every workgroup is
// cheaper than the separate quantize launch: measured at n = k = 4096, fused
// against quantize + GEMV, m = 1: 4.75 vs 6.43 us, m = 2: 6.02 vs 6.75 us; a
// fused variant of the m = 2..16 kernel took 7.6 vs 7.4 us at m = 3 and 13.9
// vs 9.4 us at m = 8.
bool fused_gemv_supported(int type, int64_t m, int64_t k) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return kquant_fused_gemv_fits(type, m, k);
    return m >= 1 && m <= 2 && k % 64 == 0 && m * (k / 32) * 34 <= 65536;
}

hipError_t launch_fused_gemv(int type, const void *w, const float *x, float *c, int64_t m, int64_t n, int64_t k,
                             hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0)
        return m == 1 ? launch_kquant_fused_gemv(type, w, x, c, n, k, stream) : hipErrorInvalidValue;
    switch (m) {
    case 1: return launch_fused_m<1>(w, x, c, n, k, stream);
    case 2: return launch_fused_m<2>(w, x, c, n, k, stream);
    default: return hipErrorInvalidValue;
    }
}

bool gemv_supported(int type, int64_t m, int64_t k) {
    if (m < 1 || k > kMaxTiledK) return false;  // 32-bit load offsets
    const bool pairs = k % 64 == 0 && pairs_lds_bytes(m, k / 32) <= kPairsMaxLds;
    if (type == PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) {
        if (m == 1) return k % 64 == 0;
        if (m <= 8) return k % 256 == 0 || pairs;
        // gemv_q4_0_mfma_chunk_kernel up to gemv_tiles_max_m(k); otherwise m = 9..16
        // in the pair-per-lane kernel
        if (m <= gemv_tiles_max_m(k) && q4_0_tiles_take_k(k)) return true;
        return m <= kPairsMaxM && pairs;
    }
    // q4_K and iq2_xxs (gemv_kquant.hip): m <= 8 for every k % 256 == 0,
    // m = 9..16 while the staged activations fit in LDS, m = 9..64 or 128 at
    // q4_K k % 1024 == 0, iq2_xxs k % 2048 == 0
    if (m > 8) return (kquant_gemv_staged_fits(m, k) || kquant_gemv_chunked_fits(type, m, k)) &&
                      (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K || type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K);
    return (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K || type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) && k % 256 == 0;
}

hipError_t launch_gemv(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                       hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_0_ACTIVATION_Q8_0) return launch_kquant_gemv(type, w, a, c, m, n, k, stream);
    switch (m) {
    case 1: {
        const int nb = (int)(k / 32);
        const size_t act_bytes = (size_t)nb * 34;
        if (act_bytes <= 65536) {
            const int grid = (int)((n + 15) / 16);
            hipLaunchKernelGGL(gemv_q4_0_m1_kernel<true>, dim3(grid), dim3(1024), act_bytes, stream,
                               static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, (int)n, nb);
        } else {
            const int grid = (int)((n + kThreads / 64 - 1) / (kThreads / 64));
            hipLaunchKernelGGL(gemv_q4_0_m1_kernel<false>, dim3(grid), dim3(kThreads), 0, stream,
                               static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, (int)n, nb);
        }
        return hipGetLastError();
    }
    case 2: return launch_gemv_q4_0_m<2>(w, a, c, n, k, stream);
    case 3: return launch_gemv_q4_0_m<3>(w, a, c, n, k, stream);
    case 4: return launch_gemv_q4_0_m<4>(w, a, c, n, k, stream);
    case 5: return launch_gemv_q4_0_m<5>(w, a, c, n, k, stream);
    case 6: return launch_gemv_q4_0_m<6>(w, a, c, n, k, stream);
    case 7: return launch_gemv_q4_0_m<7>(w, a, c, n, k, stream);
    case 8: return launch_gemv_q4_0_m<8>(w, a, c, n, k, stream);
    case 9: return launch_gemv_q4_0_m<9>(w, a, c, n, k, stream);
    case 10: return launch_gemv_q4_0_m<10>(w, a, c, n, k, stream);
    case 11: return launch_gemv_q4_0_m<11>(w, a, c, n, k, stream);
    case 12: return launch_gemv_q4_0_m<12>(w, a, c, n, k, stream);
    case 13: return launch_gemv_q4_0_m<13>(w, a, c, n, k, stream);
    case 14: return launch_gemv_q4_0_m<14>(w, a, c, n, k, stream);
    case 15: return launch_gemv_q4_0_m<15>(w, a, c, n, k, stream);
    case 16: return launch_gemv_q4_0_m<16>(w, a, c, n, k, stream);
    default: break;
    }
    if (!(m >= 17 && m <= gemv_tiles_max_m(k) && q4_0_tiles_take_k(k))) return hipErrorInvalidValue;
    const int ng = (int)(k / 256);
    const auto *wp = static_cast<const uint8_t *>(w);
    const auto *ap = static_cast<const uint8_t *>(a);
#define PFNG_Q40_CHUNK_CASE(C)                                                                                      \
    case C:                                                                                                        \
        launch_q4_0_chunk<C>(wp, ap, c, (int)m, (int)n, ng, stream);                                               \
        break;
    switch ((m + 15) / 16) {
        PFNG_Q40_CHUNK_CASE(2)
        PFNG_Q40_CHUNK_CASE(3)
        PFNG_Q40_CHUNK_CASE(4)
        PFNG_Q40_CHUNK_CASE(5)
        PFNG_Q40_CHUNK_CASE(6)
        PFNG_Q40_CHUNK_CASE(7)
        PFNG_Q40_CHUNK_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef PFNG_Q40_CHUNK_CASE
    return hipGetLastError();
}

}  // namespace pfng
