// GEMV path (m <= 16, and up to 64 or 128 for the tiles) for the super-block formats
// against q8_K activations:
// q4_K (llama_reference.cpp:113-132) and iq2_xxs (llama_reference.cpp:148-161,
// kernels/common/iq2_xxs.h:29-41). One wavefront per weight row, the weight
// stream read with aligned 16-byte (q4_K) or realigned dword (iq2_xxs,
// 66-byte blocks) loads, all loads of a step issued before any arithmetic,
// int8 dots with v_dot4_i32_i8. gemv_q4_K_kernel and gemv_iq2_xxs_kernel
// (m <= 8) take m == 1 and rows too long to stage; for q4_K at m == 1 the
// 16-row workgroups copy the activation row into LDS first. The
// *_staged_kernel variants (m = 2..16) stage the rows in LDS once per 16-row
// workgroup. At q4_K k % 1024 == 0 and iq2_xxs k % 2048 == 0 both formats run
// 16x16 int8 MFMA tiles of 16 weight rows with one super-block per wave:
// iq2_xxs at m = 5..8 and k == 4096 with the weight and activation bytes
// copied together in two halves (gemv_iq2_xxs_mfma_sb_kernel), and from
// m = kq_tiles_min_m (3..9 by format and k) with the weights decoded once per
// wave and the activation rows streamed in chunks of 16 (*_mfma_chunk_kernel;
// wave w takes super-blocks w, w + 16, ..., one per round).
//
// q4_K: four lanes per super-block, lane e owning sub-blocks 2e and 2e+1 (the
// 32 nibble bytes qs[32e .. 32e+32): low nibbles of sub-block 2e, high of
// 2e+1). Its part ad * (d * (sc_2e S_2e + sc_2e+1 S_2e+1) - dmin * (m_2e B_2e +
// m_2e+1 B_2e+1)) with B_j the two bsums of sub-block j is exact up to the
// final fp32 steps (the accuracy bound of this format is per element).
// iq2_xxs: eight lanes per super-block, one sub-block each; the eight integer
// parts (2 s_j + 1) * S_j are added across the lanes first, so the super-block
// sum is complete and exact before it is scaled by 0.125 * d * ad (the bound
// of this format is per super-block).
#include "device_common.h"
#include "kernels.h"
#include "pfng_iq2xxs_grid.h"

namespace pfng {

namespace {

constexpr int kThreads = 256;  // four rows per workgroup, one per wave
constexpr int kQ8KBytes = 292, kQ4KBytes = 144, kIq2Bytes = 66;

// The 256 grid entries expanded at compile time to their eight magnitude
// bytes (kernels/iq2_xxs-q8_K-RVV-common/ggml_min.h:69-134: two bits per byte
// select 8, 25 or 43), so a workgroup fills its LDS copy with one 8-byte load
// and store per thread.
struct alignas(16) Iq2Grid {
    uint32_t v[256][2];
};
constexpr Iq2Grid expand_iq2_grid() {
    constexpr uint16_t codes[256] = PFNG_IQ2XXS_GRID_CODES_INIT;
    Iq2Grid t{};
    for (int e = 0; e < 256; ++e)
        for (int j = 0; j < 8; ++j) {
            const uint32_t c2 = (codes[e] >> (2 * j)) & 3u;
            t.v[e][j / 4] |= (c2 == 0 ? 8u : (c2 == 1 ? 25u : 43u)) << (8 * (j % 4));
        }
    return t;
}
__constant__ Iq2Grid kIq2Grid = expand_iq2_grid();

// Sign masks: entry i is 0xff in byte j where bit j of i | parity(i) << 7 is
// set (the reference's ksigns_iq2xs, ggml_min.h:58-67, which stores exactly
// that byte, expanded to one mask byte per element).
struct alignas(16) Iq2Signs {
    uint32_t v[128][2];
};
constexpr Iq2Signs expand_iq2_signs() {
    Iq2Signs t{};
    for (int i = 0; i < 128; ++i) {
        int par = 0;
        for (int b = 0; b < 7; ++b) par ^= (i >> b) & 1;
        const int sgn = i | (par << 7);
        for (int j = 0; j < 8; ++j)
            if ((sgn >> j) & 1) t.v[i][j / 4] |= 0xffu << (8 * (j % 4));
    }
    return t;
}
__constant__ Iq2Signs kIq2Signs = expand_iq2_signs();

constexpr int kIq2TableBytes = 256 * 8 + 128 * 8;  // grid, then sign masks

// The LDS copy of both tables (384 entries of 8 bytes) for workgroups of 256
// threads, its loads and stores separate so that other loads can be issued
// between them: thread t loads entries t and t + 256 (the latter clamped into
// the table, stored only where it exists).
__device__ __forceinline__ void load_iq2_table_entries(uint32_t (&t)[4]) {
    const int e1 = (int)threadIdx.x + 256 < 384 ? (int)threadIdx.x + 256 : 383;
    t[0] = kIq2Grid.v[threadIdx.x][0];
    t[1] = kIq2Grid.v[threadIdx.x][1];
    t[2] = kIq2Signs.v[e1 - 256][0];
    t[3] = kIq2Signs.v[e1 - 256][1];
}
__device__ __forceinline__ void store_iq2_table_entries(uint8_t *tab, const uint32_t (&t)[4]) {
    *reinterpret_cast<uint2 *>(tab + 8 * threadIdx.x) = make_uint2(t[0], t[1]);
    if (threadIdx.x < 128) *reinterpret_cast<uint2 *>(tab + 8 * (threadIdx.x + 256)) = make_uint2(t[2], t[3]);
}

// Both tables as one object in the LDS layout (grid, then sign masks), for a
// wave's private copy: lane l loads and stores the 16-byte pieces l, l + 64
// and l + 128. Loads and stores are again separate steps.
struct alignas(16) Iq2Tables {
    Iq2Grid grid;
    Iq2Signs signs;
};
static_assert(sizeof(Iq2Tables) == kIq2TableBytes, "grid, then sign masks, no padding");
__constant__ Iq2Tables kIq2Tables = {expand_iq2_grid(), expand_iq2_signs()};

__device__ __forceinline__ void load_iq2_tables_wave(uint32_t (&t)[12], int lane) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const uint4 v = reinterpret_cast<const uint4 *>(&kIq2Tables)[lane + 64 * i];
        t[4 * i] = v.x;
        t[4 * i + 1] = v.y;
        t[4 * i + 2] = v.z;
        t[4 * i + 3] = v.w;
    }
}
__device__ __forceinline__ void store_iq2_tables_wave(uint8_t *tab, const uint32_t (&t)[12], int lane) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
        reinterpret_cast<uint4 *>(tab)[lane + 64 * i] = make_uint4(t[4 * i], t[4 * i + 1], t[4 * i + 2], t[4 * i + 3]);
}

// The 32 signed weights of one sub-block from its four grid indices (gidx)
// and its 28 sign-index bits plus scale nibble (ss): magnitudes are >= 8, so
// (x ^ 0xff) + 1 negates a byte without a carry into the next. kSignTable:
// the sign masks come from the LDS table (fewer VALU instructions, four more
// LDS gathers); otherwise sign bit i of group g is computed as bit i of
// idx | parity(idx) << 7 and spread over the bytes by a multiply. The table
// measured faster where the decode dominates (few activation rows), the
// arithmetic form where LDS reads of many activation rows do.
template <bool kSignTable>
__device__ __forceinline__ void iq2_decode_subblock(uint32_t gidx, uint32_t ss, const uint8_t *tab, uint32_t (&v)[8]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint2 mag = *reinterpret_cast<const uint2 *>(tab + ((gidx >> (8 * g)) & 0xffu) * 8);
        const uint32_t idx = (ss >> (7 * g)) & 0x7fu;
        if constexpr (kSignTable) {
            const uint2 neg = *reinterpret_cast<const uint2 *>(tab + 256 * 8 + idx * 8);
            v[2 * g] = (mag.x ^ neg.x) + (neg.x & 0x01010101u);
            v[2 * g + 1] = (mag.y ^ neg.y) + (neg.y & 0x01010101u);
        } else {
            const uint32_t sgn = idx | ((__builtin_popcount(idx) & 1u) << 7);
            const uint32_t s0 = ((sgn & 0xfu) * 0x00204081u) & 0x01010101u;
            const uint32_t s1 = (((sgn >> 4) & 0xfu) * 0x00204081u) & 0x01010101u;
            v[2 * g] = (mag.x ^ (s0 * 0xffu)) + s0;
            v[2 * g + 1] = (mag.y ^ (s1 * 0xffu)) + s1;
        }
    }
}

__device__ __forceinline__ int dot8(const uint32_t *w, const uint32_t *x) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = __builtin_amdgcn_sdot4((int)w[i], (int)x[i], s, false);
    return s;
}

// Scales and mins of q4_K sub-blocks 2e and 2e + 1 (e = 0..3) from the 12
// packed bytes (dwords 1..3 of the block header), the reference's decode
// (llama_reference.cpp:116-121) done four sub-blocks per dword and without a
// branch on the lane: sub-blocks 0..3 take the low six bits of bytes 0..3
// (scales) and 4..7 (mins); sub-blocks 4..7 take the low (scales) or high
// (mins) nibble of bytes 8..11 with the top two bits of bytes 0..3 (scales)
// or 4..7 (mins) above it. Lane e then picks bytes 2e % 4 and 2e % 4 + 1.
__device__ __forceinline__ void q4_K_scale_min_pair(const uint4 &hd, int e, int &sc0, int &m0, int &sc1, int &m1) {
    const uint32_t sc_lo = hd.y & 0x3f3f3f3fu, mn_lo = hd.z & 0x3f3f3f3fu;
    const uint32_t sc_hi = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
    const uint32_t scw = e < 2 ? sc_lo : sc_hi, mnw = e < 2 ? mn_lo : mn_hi;
    const int sh = 16 * (e & 1);
    sc0 = (int)((scw >> sh) & 0xffu);
    sc1 = (int)((scw >> (sh + 8)) & 0xffu);
    m0 = (int)((mnw >> sh) & 0xffu);
    m1 = (int)((mnw >> (sh + 8)) & 0xffu);
}

// kLdsAct (m == 1, rows up to 64 KB): workgroups of 16 weight rows copy the
// activation row into LDS once, and the waves read it there instead of each
// fetching it from L2. The copy uses direct loads into LDS
// (global_load_lds_dwordx4: lane i of a wave writes 16 bytes at the wave's
// LDS base + 16 i), and every lane issues the three 16-byte loads of its
// first weight step (clamped, so always issued) before any wave waits: each
// wave then waits for its own copies only (s_waitcnt vmcnt(3): memory loads
// complete in issue order) and meets the others at the barrier, so the
// activation's trip from L2 overlaps the weight stream.
// kQuantAct (fused activation quantization, with kLdsAct): a_global is the
// fp32 activation row instead, and the workgroup quantizes it into q8_K blocks
// in LDS (wave w taking blocks w, w + 16, ...) with the quantize kernel's
// arithmetic, so the bytes and the outputs equal the separate quantize + GEMV.
constexpr int kM1LdsThreads = 1024;

template <int M, bool kLdsAct = false, bool kQuantAct = false>
__global__ __launch_bounds__(kLdsAct ? kM1LdsThreads : kThreads) void gemv_q4_K_kernel(
    const uint8_t *__restrict__ w, const uint8_t *__restrict__ a_global, float *__restrict__ c, int n, int nb) {
    static_assert(!kQuantAct || kLdsAct, "the quantized row lives in LDS");
    constexpr int kBlockThreads = kLdsAct ? kM1LdsThreads : kThreads;
    extern __shared__ __align__(16) uint8_t sact[];
    const int lane = threadIdx.x & 63;
    // the row is uniform across the wave: its base address lives in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = blockIdx.x * (kBlockThreads / 64) + wave;
    const int lrow = row < n ? row : n - 1;  // clamped: loads stay unconditional, the store is guarded
    const uint8_t *wrow = w + (size_t)lrow * nb * kQ4KBytes;
    const int slot = lane >> 2, e = lane & 3;
    // lane's header and 32 nibble bytes of super-block b0 + slot (clamped)
    auto load_w = [&](int b0, uint4 (&wq)[3]) {
        const int b = b0 + slot;
        const uint8_t *blk = wrow + (uint32_t)(b < nb ? b : nb - 1) * (uint32_t)kQ4KBytes;
        wq[0] = *reinterpret_cast<const uint4 *>(blk);
        wq[1] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * e);
        wq[2] = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * e);
    };
    float acc[M];
#pragma unroll
    for (int mi = 0; mi < M; ++mi) acc[mi] = 0.0f;
    // acc += the step's super-block parts against activations a
    auto step = [&](int b0, const uint4 (&wq)[3], const uint8_t *a) {
        const int b = b0 + slot;
        const bool valid = b < nb;
        const int lb = valid ? b : nb - 1;
        uint32_t x[M][16], bs[M][2];
        float ad[M];
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            const uint8_t *ab = a + ((size_t)mi * nb + lb) * kQ8KBytes;
            const uint32_t *xs = reinterpret_cast<const uint32_t *>(ab + 4 + 64 * e);
#pragma unroll
            for (int i = 0; i < 16; ++i) x[mi][i] = xs[i];
            const uint32_t *bp = reinterpret_cast<const uint32_t *>(ab + 260 + 8 * e);
            bs[mi][0] = bp[0];
            bs[mi][1] = bp[1];
            ad[mi] = *reinterpret_cast<const float *>(ab);
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint4 &hd = wq[0], &qa = wq[1], &qb = wq[2];
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            lo[i] = q[i] & 0x0f0f0f0fu;
            hi[i] = (q[i] >> 4) & 0x0f0f0f0fu;
        }
        int sc0, m0, sc1, m1;
        q4_K_scale_min_pair(hd, e, sc0, m0, sc1, m1);
        const float d = fp16_to_f32(hd.x & 0xffffu), dmin = fp16_to_f32(hd.x >> 16);
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            const int is = sc0 * dot8(lo, x[mi]) + sc1 * dot8(hi, x[mi] + 8);
            const int b0s = (int)(int16_t)(bs[mi][0] & 0xffffu) + (int)(int16_t)(bs[mi][0] >> 16);
            const int b1s = (int)(int16_t)(bs[mi][1] & 0xffffu) + (int)(int16_t)(bs[mi][1] >> 16);
            const int im = m0 * b0s + m1 * b1s;
            const float part = ad[mi] * fmaf(-dmin, (float)im, d * (float)is);
            acc[mi] += valid ? part : 0.0f;
        }
    };
    int b0 = 0;
    const uint8_t *a = a_global;
    if constexpr (kQuantAct) {
        static_assert(M == 1, "one activation row");
        constexpr int kWaves = kBlockThreads / 64;
        const float *x = reinterpret_cast<const float *>(a_global);
        // the first block's elements, then the first weight step: the
        // quantization waits for its own loads only
        float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (wave < nb) v0 = *reinterpret_cast<const float4 *>(x + (size_t)wave * 256 + lane * 4);
        __builtin_amdgcn_sched_barrier(0);
        uint4 wq[3];
        load_w(0, wq);
        __builtin_amdgcn_sched_barrier(0);
        if (wave < nb) q8_K_store_lane(sact + wave * kQ8KBytes, q8_K_quantize_lane(v0), lane);
        for (int b = wave + kWaves; b < nb; b += kWaves)
            q8_K_store_lane(sact + b * kQ8KBytes,
                            q8_K_quantize_lane(*reinterpret_cast<const float4 *>(x + (size_t)b * 256 + lane * 4)),
                            lane);
        __syncthreads();
        a = sact;
        step(0, wq, a);
        b0 = 16;
    } else if constexpr (kLdsAct) {
        static_assert(M == 1, "one activation row");
        // 16-byte chunks (the row base is 16-byte aligned), wave w taking
        // chunks 64 w + lane (+ 1024 per round), then the dword tail from the
        // last wave
        const int n16 = nb * kQ8KBytes / 16, nd = nb * kQ8KBytes / 4;
        for (int c0 = wave * 64; c0 < n16; c0 += kBlockThreads) {
            if (c0 + lane < n16)
                __builtin_amdgcn_global_load_lds(a_global + (size_t)(c0 + lane) * 16,
                                                 (__attribute__((address_space(3))) void *)(sact + c0 * 16), 16, 0, 0);
        }
        if (wave == kBlockThreads / 64 - 1 && 4 * n16 + lane < nd)
            __builtin_amdgcn_global_load_lds(a_global + (size_t)(4 * n16 + lane) * 4,
                                             (__attribute__((address_space(3))) void *)(sact + n16 * 16), 4, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        uint4 wq[3];
        load_w(0, wq);
        asm volatile("s_waitcnt vmcnt(3)\n\ts_barrier" ::: "memory");
        a = sact;
        step(0, wq, a);
        b0 = 16;
    }
    for (; b0 < nb; b0 += 16) {
        uint4 wq[3];
        load_w(b0, wq);
        step(b0, wq, a);
    }
#pragma unroll
    for (int mi = 0; mi < M; ++mi) acc[mi] = wave_sum_lane63(acc[mi]);
    if (row < n && lane == 63) {
#pragma unroll
        for (int mi = 0; mi < M; ++mi) c[(size_t)mi * n + row] = acc[mi];
    }
}

// Each wave copies both tables into its own LDS region (3 KB a wave) and
// reads only that copy, so no wave waits at a workgroup barrier for the
// others' copies: a wave issues its table loads, then the first step's loads,
// stores the table (waiting for the table loads only) and decodes as soon as
// its own weights are in. Against one shared copy behind a barrier: 3.72 ->
// 3.55 us at 4096 x 4096, the same bits (4 or 8 waves a workgroup alike, 16
// waves 3.61 us).
template <int M>
__global__ __launch_bounds__(kThreads) void gemv_iq2_xxs_kernel(const uint8_t *__restrict__ w,
                                                               const uint8_t *__restrict__ a, float *__restrict__ c,
                                                               int n, int nb) {
    __shared__ __align__(16) uint8_t tables[(kThreads / 64) * kIq2TableBytes];
    const int lane = threadIdx.x & 63;
    // the table's address is fixed at load time: its loads go out first,
    // before anything that needs a kernel argument (where the arguments are
    // loaded rather than preloaded, before the wave waits for them: 3.55
    // against 3.85 us when issued after that wait)
    uint32_t tab[12];
    load_iq2_tables_wave(tab, lane);
    __builtin_amdgcn_sched_barrier(0);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    uint8_t *const grid = tables + wave * kIq2TableBytes;
    const int row = blockIdx.x * (kThreads / 64) + wave;
    const int lrow = row < n ? row : n - 1;
    const int slot = lane >> 3, j = lane & 7;
    // the row's base once; per step only the block offset
    const size_t wbase = (size_t)lrow * nb * kIq2Bytes;
    const uint8_t *wrow = w + wbase;
    // one step's loads: the lane's sub-block words (66-byte blocks are 2-byte
    // aligned: the covering dwords plus a trailing half-word, never past the
    // sub-block's last byte), the block's d, and then the activation
    // sub-blocks, in that order (fixed by a scheduling fence; the decode,
    // which needs the weight words only, then waits for them alone; the
    // other order measured the same)
    struct Step {
        uint32_t wv[2];  // d0, d1
        uint16_t th[2];  // tail, dh (widened when decoded)
        uint32_t x[M][8];
        float ad[M];
    };
    auto load = [&](int b0, Step &st) {
        const int b = b0 + slot;
        const int lb = b < nb ? b : nb - 1;
        const size_t boff = (size_t)lb * kIq2Bytes;
        const size_t o = boff + 2 + 8 * j;
        const bool sh = ((wbase + o) & 3) != 0;
        const uint32_t *p4 = reinterpret_cast<const uint32_t *>(wrow + o - (sh ? 2 : 0));
        st.wv[0] = p4[0];
        st.wv[1] = p4[1];
        st.th[0] = *reinterpret_cast<const uint16_t *>(wrow + o + 6);
        st.th[1] = *reinterpret_cast<const uint16_t *>(wrow + boff);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            const uint8_t *ab = a + (size_t)(mi * nb + lb) * kQ8KBytes;
            const uint32_t *xs = reinterpret_cast<const uint32_t *>(ab + 4 + 32 * j);
#pragma unroll
            for (int i = 0; i < 8; ++i) st.x[mi][i] = xs[i];
            st.ad[mi] = *reinterpret_cast<const float *>(ab);
        }
    };
    float acc[M];
#pragma unroll
    for (int mi = 0; mi < M; ++mi) acc[mi] = 0.0f;
    auto compute = [&](int b0, const Step &st) {
        const int b = b0 + slot;
        const bool valid = b < nb;
        const int lb = valid ? b : nb - 1;
        const bool sh = ((wbase + (size_t)lb * kIq2Bytes + 2 + 8 * j) & 3) != 0;
        const uint32_t d0 = st.wv[0], d1 = st.wv[1], tail = st.th[0], dh = st.th[1];
        const uint32_t gidx = sh ? __builtin_amdgcn_alignbyte(d1, d0, 2) : d0;
        const uint32_t ss = sh ? ((d1 >> 16) | (tail << 16)) : d1;
        uint32_t v[8];
        iq2_decode_subblock<true>(gidx, ss, grid, v);
        const int scale = 2 * (int)(ss >> 28) + 1;
        const float t0 = 0.125f * fp16_to_f32(dh);
#pragma unroll
        for (int mi = 0; mi < M; ++mi) {
            // exact integer sum of the super-block over its eight lanes
            const int is = group_sum_dpp<8>(scale * dot8(v, st.x[mi]));
            if (j == 0 && valid) acc[mi] += (t0 * st.ad[mi]) * (float)is;
        }
    };
    Step st0;
    load(0, st0);
    __builtin_amdgcn_sched_barrier(0);
    use_here(tab);
    store_iq2_tables_wave(grid, tab, lane);
    redefine_here(st0.wv);  // decoded after the table stores
    redefine_here(st0.th);
    compute(0, st0);
    for (int b0 = 8; b0 < nb; b0 += 8) {
        Step st;
        load(b0, st);
        __builtin_amdgcn_sched_barrier(0);
        compute(b0, st);
    }
#pragma unroll
    for (int mi = 0; mi < M; ++mi) acc[mi] = wave_sum_lane63(acc[mi]);
    if (row < n && lane == 63) {
#pragma unroll
        for (int mi = 0; mi < M; ++mi) c[(size_t)mi * n + row] = acc[mi];
    }
}

// Fused activation quantization + GEMV for iq2_xxs at m == 1: WAVES weight
// rows per workgroup (one per wave). The workgroup copies the grid and sign
// tables into LDS and quantizes the fp32 activation row into q8_K blocks
// behind them (wave w taking blocks w, w + WAVES, ...; the quantize kernel's
// arithmetic, so the bytes equal the standalone quantizer's); the weight words
// of the first two steps are loaded before either, so their trip from HBM
// overlaps both. Per step as gemv_iq2_xxs_kernel<1>, the activations read from
// LDS; the sums are formed in the same order, so the outputs equal the
// separate quantize + GEMV bit for bit.
template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_iq2_xxs_fused_kernel(const uint8_t *__restrict__ w,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ c, int n, int nb) {
    constexpr int kBlock = WAVES * 64;
    static_assert(kBlock == 256 || kBlock >= 384, "table copy: two entries per thread or one");
    extern __shared__ __align__(16) uint8_t lds[];  // tables, then nb q8_K blocks
    uint8_t *const grid = lds;
    uint8_t *const aq = lds + kIq2TableBytes;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row = blockIdx.x * WAVES + wave;
    const int lrow = row < n ? row : n - 1;
    const int slot = lane >> 3, j = lane & 7;
    const size_t wbase = (size_t)lrow * nb * kIq2Bytes;
    const uint8_t *wrow = w + wbase;
    struct WStep {
        uint32_t wv[2];
        uint16_t th[2];
    };
    auto load = [&](int b0, WStep &st) {
        const int b = b0 + slot;
        const int lb = b < nb ? b : nb - 1;
        const size_t boff = (size_t)lb * kIq2Bytes;
        const size_t o = boff + 2 + 8 * j;
        const bool sh = ((wbase + o) & 3) != 0;
        const uint32_t *p4 = reinterpret_cast<const uint32_t *>(wrow + o - (sh ? 2 : 0));
        st.wv[0] = p4[0];
        st.wv[1] = p4[1];
        st.th[0] = *reinterpret_cast<const uint16_t *>(wrow + o + 6);
        st.th[1] = *reinterpret_cast<const uint16_t *>(wrow + boff);
    };
    float acc = 0.0f;
    auto compute = [&](int b0, const WStep &st) {
        const int b = b0 + slot;
        const bool valid = b < nb;
        const int lb = valid ? b : nb - 1;
        const bool sh = ((wbase + (size_t)lb * kIq2Bytes + 2 + 8 * j) & 3) != 0;
        const uint32_t d0 = st.wv[0], d1 = st.wv[1], tail = st.th[0], dh = st.th[1];
        const uint32_t gidx = sh ? __builtin_amdgcn_alignbyte(d1, d0, 2) : d0;
        const uint32_t ss = sh ? ((d1 >> 16) | (tail << 16)) : d1;
        const uint8_t *ab = aq + lb * kQ8KBytes;
        const uint32_t *xs = reinterpret_cast<const uint32_t *>(ab + 4 + 32 * j);
        uint32_t xv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = xs[i];
        const float ad = *reinterpret_cast<const float *>(ab);
        uint32_t v[8];
        iq2_decode_subblock<true>(gidx, ss, grid, v);
        const int scale = 2 * (int)(ss >> 28) + 1;
        const float t0 = 0.125f * fp16_to_f32(dh);
        const int is = group_sum_dpp<8>(scale * dot8(v, xv));
        if (j == 0 && valid) acc += (t0 * ad) * (float)is;
    };
    // table entries, the first block's elements and the first two weight
    // steps go out before any arithmetic
    uint32_t tab[4];
    if constexpr (kBlock == 256) {
        load_iq2_table_entries(tab);
    } else {
        const int e = (int)threadIdx.x < 384 ? (int)threadIdx.x : 383;
        tab[0] = e < 256 ? kIq2Grid.v[e][0] : kIq2Signs.v[e - 256][0];
        tab[1] = e < 256 ? kIq2Grid.v[e][1] : kIq2Signs.v[e - 256][1];
    }
    float4 v0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (wave < nb) v0 = *reinterpret_cast<const float4 *>(x + (size_t)wave * 256 + lane * 4);
    __builtin_amdgcn_sched_barrier(0);
    WStep st[2];
    load(0, st[0]);
    if (nb > 8) load(8, st[1]);  // uniform
    __builtin_amdgcn_sched_barrier(0);
    use_here(tab);
    if constexpr (kBlock == 256) {
        store_iq2_table_entries(grid, tab);
    } else if ((int)threadIdx.x < 384) {
        *reinterpret_cast<uint2 *>(grid + 8 * threadIdx.x) = make_uint2(tab[0], tab[1]);
    }
    if (wave < nb) q8_K_store_lane(aq + wave * kQ8KBytes, q8_K_quantize_lane(v0), lane);
    for (int b = wave + WAVES; b < nb; b += WAVES)
        q8_K_store_lane(aq + b * kQ8KBytes,
                        q8_K_quantize_lane(*reinterpret_cast<const float4 *>(x + (size_t)b * 256 + lane * 4)), lane);
    __syncthreads();
    for (int b0 = 0; b0 < nb; b0 += 16) {
        // decoded after the barrier, which then waits for the tables and the
        // quantization only
        redefine_here(st[0].wv);
        redefine_here(st[0].th);
        compute(b0, st[0]);
        __builtin_amdgcn_sched_barrier(0);
        if (b0 + 16 < nb) load(b0 + 16, st[0]);
        if (b0 + 8 < nb) {
            redefine_here(st[1].wv);
            redefine_here(st[1].th);
            compute(b0 + 8, st[1]);
            __builtin_amdgcn_sched_barrier(0);
            if (b0 + 24 < nb) load(b0 + 24, st[1]);
        }
    }
    acc = wave_sum_lane63(acc);
    if (row < n && lane == 63) c[row] = acc;
}

// ---------------------------------------------------------------------------
// m = 2..8 with the q8_K activation rows staged in LDS once per workgroup of
// 16 weight rows (one per wavefront): each 292-byte block becomes 256 int8
// bytes at a 272-byte stride (16-byte aligned for ds_read_b128, staggered
// over the banks) and a 48-byte side record with the eight per-sub-block bsum
// pairs bsums[2j] + bsums[2j+1] as int32 and d as fp32. The waves then read
// activations from LDS instead of issuing 16-19 dword loads per row each.
// Cross-lane sums use the reduce-scatter of gemv_q4_0_pairs_kernel: P
// accumulators hold activation row q ^ f(lane), so every lane keeps the lower
// half of each exchange and accumulators are only indexed by constants. P is
// the largest power of two <= m (the other m - P rows take a plain butterfly)
// or, where that measured faster, the next power of two (accumulators of rows
// >= m read a clamped row, combine only with each other, are never stored).
constexpr int kStagedThreads = 1024;
constexpr int kQsStride = 272, kSideStride = 48;

__host__ __device__ constexpr int64_t kq_staged_lds_bytes(int64_t m, int64_t nsb) {
    return m * nsb * (kQsStride + kSideStride) + kIq2TableBytes;  // + the iq2_xxs tables
}

// Four tasks per block: quarter t copies qs[64t, 64t + 64), forms the bsum
// pairs 2t and 2t + 1, and quarter 0 also copies d (fp32 already). A task's
// loads (16 qs dwords, two bsum dwords, d) and its LDS stores are separate
// steps, so that a kernel can issue other loads between them.
__device__ __forceinline__ void load_q8_K_quarter(const uint8_t *__restrict__ a, int task, uint32_t (&r)[19]) {
    const int blk = task >> 2, t = task & 3;
    const uint8_t *src = a + (size_t)blk * kQ8KBytes;
    const uint32_t *q = reinterpret_cast<const uint32_t *>(src + 4 + 64 * t);
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = q[i];
    const uint32_t *bp = reinterpret_cast<const uint32_t *>(src + 260 + 8 * t);
    r[16] = bp[0];
    r[17] = bp[1];
    r[18] = *reinterpret_cast<const uint32_t *>(src);
}
__device__ __forceinline__ void store_q8_K_quarter(uint8_t *qs, uint8_t *side, int task, const uint32_t (&r)[19]) {
    const int blk = task >> 2, t = task & 3;
    uint4 *dq = reinterpret_cast<uint4 *>(qs + (size_t)blk * kQsStride + 64 * t);
#pragma unroll
    for (int i = 0; i < 4; ++i) dq[i] = make_uint4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
    uint8_t *sd = side + (size_t)blk * kSideStride;
    *reinterpret_cast<int2 *>(sd + 8 * t) = make_int2((int)(int16_t)(r[16] & 0xffffu) + (int)(int16_t)(r[16] >> 16),
                                                      (int)(int16_t)(r[17] & 0xffffu) + (int)(int16_t)(r[17] >> 16));
    if (t == 0) *reinterpret_cast<uint32_t *>(sd + 32) = r[18];
}

// The staging prologue shared by the staged kernels: each thread loads its
// first staging task (the only one while m * k / 64 <= 1024, so always at
// k <= 4096; threads without one load nothing) and then calls issue(), which
// issues the loads of the lane's first weight step; only then are the first
// tasks stored (waiting for their own loads) and the remaining tasks staged.
// The caller's barrier then waits for the staging alone, and the weights'
// trip from HBM overlaps it.
template <int M, class Issue>
__device__ __forceinline__ void stage_q8_K_overlapped(const uint8_t *__restrict__ a, uint8_t *qs, uint8_t *side, int nsb,
                                                      Issue issue) {
    const int ntask = M * nsb * 4;
    int task = threadIdx.x;
    uint32_t r0[19];
    if (task < ntask) {
        load_q8_K_quarter(a, task, r0);
    } else {
#pragma unroll
        for (int i = 0; i < 19; ++i) r0[i] = 0;
    }
    __builtin_amdgcn_sched_barrier(0);
    issue();
    __builtin_amdgcn_sched_barrier(0);
    use_here(r0);
    if (task < ntask) store_q8_K_quarter(qs, side, task, r0);
    for (task += kStagedThreads; task < ntask; task += kStagedThreads) {
        uint32_t r[19];
        load_q8_K_quarter(a, task, r);
        store_q8_K_quarter(qs, side, task, r);
    }
}

// q4_K: four lanes per super-block as gemv_q4_K_kernel, 16 super-blocks per
// wave and step.
template <int M>
__global__ __launch_bounds__(kStagedThreads) void gemv_q4_K_staged_kernel(const uint8_t *__restrict__ w,
                                                                         const uint8_t *__restrict__ a,
                                                                         float *__restrict__ c, int n, int nb) {
    // reduce-scatter width: padded to the next power of two at M = 7 and
    // M >= 13 (dummy rows, never stored), where that measured faster
    constexpr int P = M == 7 || M >= 13 ? pow2_ceil16(M) : pow2_floor16(M);
    constexpr int NA = P > M ? P : M;  // accumulators per lane
    constexpr int kLaneShift = 6 - log2_pow2(P);
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *qs = lds, *side = lds + (size_t)M * nb * kQsStride;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kStagedThreads / 64) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lrow = row < n ? row : n - 1;  // clamped: loads stay unconditional, the store is guarded
    const uint8_t *wrow = w + (size_t)lrow * nb * kQ4KBytes;
    const int slot = lane >> 2, e = lane & 3;
    const int f = lane >> kLaneShift;
    // the lane's header and 32 nibble bytes of super-block b0 + slot (clamped)
    auto load_w = [&](int b0, uint32_t (&wq)[12]) {
        const int b = b0 + slot;
        const uint8_t *blk = wrow + (uint32_t)(b < nb ? b : nb - 1) * (uint32_t)kQ4KBytes;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * e);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * e);
        const uint32_t t[12] = {hd.x, hd.y, hd.z, hd.w, qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int i = 0; i < 12; ++i) wq[i] = t[i];
    };
    float acc[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) acc[q] = 0.0f;
    auto step = [&](int b0, const uint32_t (&wq)[12]) {
        const int b = b0 + slot;
        const bool valid = b < nb;
        const int lb = valid ? b : nb - 1;
        const uint4 hd = make_uint4(wq[0], wq[1], wq[2], wq[3]);
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            lo[i] = wq[4 + i] & 0x0f0f0f0fu;
            hi[i] = (wq[4 + i] >> 4) & 0x0f0f0f0fu;
        }
        int sc0, m0, sc1, m1;
        q4_K_scale_min_pair(hd, e, sc0, m0, sc1, m1);
        const float d = fp16_to_f32(hd.x & 0xffffu), dmin = fp16_to_f32(hd.x >> 16);
#pragma unroll
        for (int q = 0; q < NA; ++q) {
            const int r0 = q < P ? q ^ f : q;
            const int rec = (r0 < M ? r0 : M - 1) * nb + lb;
            const uint4 *xq = reinterpret_cast<const uint4 *>(qs + (size_t)rec * kQsStride + 64 * e);
            uint32_t x[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 t = xq[i];
                x[4 * i] = t.x;
                x[4 * i + 1] = t.y;
                x[4 * i + 2] = t.z;
                x[4 * i + 3] = t.w;
            }
            const uint8_t *sd = side + (size_t)rec * kSideStride;
            const int2 bsp = *reinterpret_cast<const int2 *>(sd + 8 * e);
            const float ad = *reinterpret_cast<const float *>(sd + 32);
            const int is = sc0 * dot8(lo, x) + sc1 * dot8(hi, x + 8);
            const int im = m0 * bsp.x + m1 * bsp.y;
            const float part = ad * fmaf(-dmin, (float)im, d * (float)is);
            acc[q] += valid ? part : 0.0f;
        }
    };
    uint32_t wq0[12];
    stage_q8_K_overlapped<M>(a, qs, side, nb, [&] { load_w(0, wq0); });
    __syncthreads();
    redefine_here(wq0);  // decoded after the barrier, which then waits for the staging only
    step(0, wq0);
    for (int b0 = 16; b0 < nb; b0 += 16) {
        uint32_t wq[12];
        load_w(b0, wq);
        __builtin_amdgcn_sched_barrier(0);
        step(b0, wq);
    }
    // reduce-scatter (exchange offsets 32, 16, ...), then a DPP sum over the
    // 64 / P lanes left: the group's last lane holds it
    constexpr int G = 1 << kLaneShift;
    reduce_scatter_steps<P / 2, 32>(acc);
    acc[0] = group_sum_dpp<G>(acc[0]);
#pragma unroll
    for (int q = P; q < M; ++q) acc[q] = wave_sum_lane63(acc[q]);
    if (row < n) {
        if ((lane & (G - 1)) == G - 1 && f < M) c[(size_t)f * n + row] = acc[0];
        if (lane == 63) {
#pragma unroll
            for (int q = P; q < M; ++q) c[(size_t)q * n + row] = acc[q];
        }
    }
}

// iq2_xxs: eight lanes per super-block as gemv_iq2_xxs_kernel, eight
// super-blocks per wave and step. The integer super-block sums are completed
// across the eight lanes before any scaling (the bound of this format is per
// super-block). Rows go in NG groups of P: accumulator q < NG * P of lane j
// holds activation row P * (q / P) + ((q % P) ^ (j % P)), a reduce-scatter
// over the low lane bits leaves lane j with the exact sum of row
// P * g + j % P of each group g, and lanes j < P scale it once. With one group
// the rows past P (if any) take a plain butterfly each.
template <int M>
__global__ __launch_bounds__(kStagedThreads) void gemv_iq2_xxs_staged_kernel(const uint8_t *__restrict__ w,
                                                                            const uint8_t *__restrict__ a,
                                                                            float *__restrict__ c, int n, int nb) {
    // groups of 8 rows above M = 8; up to 8, one group padded to 8 from M = 6
    // on (dummy rows, never stored), where that measured faster than
    // per-step butterflies of the rows past the largest power of two
    constexpr int NG = (M + 7) / 8;
    constexpr int P = NG > 1 || M >= 6 ? 8 : pow2_floor16(M);
    constexpr int NX = NG * P < M ? M - NG * P : 0;  // rows past the groups (one group only)
    constexpr int NA = NG * P + NX;
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t *qs = lds, *side = lds + (size_t)M * nb * kQsStride;
    uint8_t *grid = side + (size_t)M * nb * kSideStride;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kStagedThreads / 64) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lrow = row < n ? row : n - 1;
    const size_t wbase = (size_t)lrow * nb * kIq2Bytes;  // offsets from w, which is 4-byte aligned
    const uint8_t *wrow = w + wbase;
    const int slot = lane >> 3, j = lane & 7;
    const int f = j & (P - 1);
    // 66-byte blocks are 2-byte aligned: the covering dwords plus a trailing
    // half-word, never past the sub-block's last byte; wv = d0, d1, th = tail,
    // dh (kept 16-bit until decoded)
    auto load_w = [&](int b0, uint32_t (&wv)[2], uint16_t (&th)[2]) {
        const int b = b0 + slot;
        const size_t boff = (size_t)(b < nb ? b : nb - 1) * kIq2Bytes;
        const size_t o = boff + 2 + 8 * j;
        const bool sh = ((wbase + o) & 3) != 0;
        const uint32_t *p4 = reinterpret_cast<const uint32_t *>(wrow + o - (sh ? 2 : 0));
        wv[0] = p4[0];
        wv[1] = p4[1];
        th[0] = *reinterpret_cast<const uint16_t *>(wrow + o + 6);
        th[1] = *reinterpret_cast<const uint16_t *>(wrow + boff);
    };
    float accp[NG];               // row P * g + f, in lanes j < P
    float accx[NX > 0 ? NX : 1];  // rows NG * P.., in lanes j == 0
#pragma unroll
    for (int g = 0; g < NG; ++g) accp[g] = 0.0f;
#pragma unroll
    for (int q = 0; q < (NX > 0 ? NX : 1); ++q) accx[q] = 0.0f;
    auto step = [&](int b0, const uint32_t (&wv)[2], const uint16_t (&th)[2]) {
        const int b = b0 + slot;
        const bool valid = b < nb;
        const int lb = valid ? b : nb - 1;
        const bool sh = ((wbase + (size_t)lb * kIq2Bytes + 2 + 8 * j) & 3) != 0;
        const uint32_t d0 = wv[0], d1 = wv[1], tail = th[0], dh = th[1];
        const uint32_t gidx = sh ? __builtin_amdgcn_alignbyte(d1, d0, 2) : d0;
        const uint32_t ss = sh ? ((d1 >> 16) | (tail << 16)) : d1;
        uint32_t v[8];
        iq2_decode_subblock<(M <= 4)>(gidx, ss, grid, v);
        const int scale = 2 * (int)(ss >> 28) + 1;
        const float t0 = valid ? 0.125f * fp16_to_f32(dh) : 0.0f;
        int is[NA];
#pragma unroll
        for (int q = 0; q < NA; ++q) {
            const int r0 = q < NG * P ? P * (q / P) + ((q % P) ^ f) : q;
            const int r = r0 < M ? r0 : M - 1;
            const uint4 *xq = reinterpret_cast<const uint4 *>(qs + (size_t)(r * nb + lb) * kQsStride + 32 * j);
            const uint4 x0 = xq[0], x1 = xq[1];
            const uint32_t x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            is[q] = scale * dot8(v, x);
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            // exact integer sums over the eight lanes of the super-block
            if (g == 0) reduce_scatter_steps<P / 2, P / 2, 0>(is);
            if constexpr (NG > 1)
                if (g == 1) reduce_scatter_steps<P / 2, P / 2, P>(is);
            if constexpr (P <= 2) is[P * g] += xor_shfl<2>(is[P * g]);
            if constexpr (P <= 4) is[P * g] += xor_shfl<4>(is[P * g]);
            const int rp = P * g + f;
            const float adp = *reinterpret_cast<const float *>(
                side + (size_t)((rp < M ? rp : M - 1) * nb + lb) * kSideStride + 32);
            if (j < P) accp[g] += (t0 * adp) * (float)is[P * g];
        }
#pragma unroll
        for (int q = NG * P; q < NA; ++q) {
            const int tot = group_sum_dpp<8>(is[q]);
            const float adq = *reinterpret_cast<const float *>(side + (size_t)(q * nb + lb) * kSideStride + 32);
            if (j == 0) accx[q - NG * P] += (t0 * adq) * (float)tot;
        }
    };
    // the table entry of this thread (384 entries, one per thread) is loaded
    // with the first staging task, ahead of the weights
    static_assert(kStagedThreads >= 384, "one table entry per thread");
    const int te = (int)threadIdx.x < 384 ? (int)threadIdx.x : 383;
    const uint32_t *tsrc = te < 256 ? kIq2Grid.v[te] : kIq2Signs.v[te - 256];
    uint32_t tab[2] = {tsrc[0], tsrc[1]};
    // kPrefetch (one group of rows): the first two steps' weights (the whole
    // row at k = 4096; clamped, so a step past the end reloads the last
    // block) go out with the staging, and every later step's one step ahead
    // of its arithmetic; measured 2 % faster at M = 8, 1 % slower at M = 16
    constexpr bool kPrefetch = NG == 1;
    uint32_t wv0[2], wv1[2];
    uint16_t th0[2], th1[2];
    stage_q8_K_overlapped<M>(a, qs, side, nb, [&] {
        load_w(0, wv0, th0);
        if constexpr (kPrefetch) load_w(8, wv1, th1);
    });
    use_here(tab);
    if (threadIdx.x < 384) *reinterpret_cast<uint2 *>(grid + 8 * threadIdx.x) = make_uint2(tab[0], tab[1]);
    __syncthreads();
    redefine_here(wv0);  // decoded after the barrier, which then waits for the staging only
    redefine_here(th0);
    if constexpr (kPrefetch) {
        redefine_here(wv1);
        redefine_here(th1);
    }
    step(0, wv0, th0);
    for (int b0 = 8; b0 < nb; b0 += 8) {
        if constexpr (kPrefetch) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                wv0[i] = wv1[i];
                th0[i] = th1[i];
            }
            if (b0 + 8 < nb) load_w(b0 + 8, wv1, th1);
        } else {
            load_w(b0, wv0, th0);
        }
        __builtin_amdgcn_sched_barrier(0);
        step(b0, wv0, th0);
    }
    // across the eight super-block slots
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        accp[g] += xor_shfl<8>(accp[g]);
        accp[g] += xor_shfl<16>(accp[g]);
        accp[g] += xor_shfl<32>(accp[g]);
    }
#pragma unroll
    for (int q = 0; q < NX; ++q) accx[q] = wave_sum_lane63(accx[q]);
    if (row < n) {
#pragma unroll
        for (int g = 0; g < NG; ++g)
            if (lane < P && P * g + lane < M) c[(size_t)(P * g + lane) * n + row] = accp[g];
        if (lane == 63) {
#pragma unroll
            for (int q = 0; q < NX; ++q) c[(size_t)(NG * P + q) * n + row] = accx[q];
        }
    }
}

// the MFMA tile GEMVs below run 16 waves per workgroup
constexpr int kKqMfWaves = 16;

// Two-half copies for the iq2_xxs GEMV with one super-block per wave
// (k == 4096, m = 5..8). A wave copies its super-block of the tile's 16 weight rows and
// of the m activation rows in 16-byte chunks, each row from the 16-byte
// boundary at or before its block (rows are 16 blocks long, so that offset
// depends on the wave only). Half h holds, for each weight row, chunks
// [wc_h, wc_h + wn_h) of the row's copy, then, for each activation row, chunks
// [ac_h, ac_h + an_h) (wc_0 = ac_0 = 0). Half 1 starts one chunk before the end
// of half 0 so that no value straddles the halves, and every row length is an
// odd number of chunks: rows whose LDS stride is 16 bytes times an odd number
// put the 16 rows of a tile on 8 different bank groups (2-way conflicts at
// most, against up to 16-way for strides of 8 chunks). The chunks of both halves
// are one flat run in LDS, copied 64 per instruction with every lane active:
// lanes past the last chunk repeat it into a pad, so no lane is predicated (a
// predicated direct-to-LDS copy may be merged by the compiler into one whose
// LDS address comes from a single lane). Loads complete in issue order, so a
// wave multiplies half 0 after waiting for the instructions that wrote it,
// while half 1 is still in flight.
struct Iq2Run {  // 66-byte weight blocks; no bsums needed
    static constexpr int wn0 = 3, wc1 = 2, wn1 = 3, an0 = 9, ac1 = 8, an1 = 9;
    static constexpr uint32_t wrow = 16 * kIq2Bytes, arow = 16 * kQ8KBytes;
};

template <class R> __host__ __device__ constexpr int sb_half0(int m) { return 16 * R::wn0 + m * R::an0; }
template <class R> __host__ __device__ constexpr int sb_half1(int m) { return 16 * R::wn1 + m * R::an1; }
template <class R> __host__ __device__ constexpr int sb_copies(int m) { return (sb_half0<R>(m) + sb_half1<R>(m) + 63) / 64; }

// Byte offset of LDS chunk p of a wave's run: from the copy start of the
// wave's block in the tile's first weight row, or (bit 31 set) in activation
// row 0. Rows past the last weight row repeat it.
template <class R, int M>
__device__ __forceinline__ uint32_t sb_chunk(int p, int rows) {
    constexpr int kH0 = sb_half0<R>(M), kH1 = sb_half1<R>(M);
    if (p >= kH0 + kH1) p = kH0 + kH1 - 1;
    uint32_t off;
    if (p < 16 * R::wn0) {
        const int row = p / R::wn0;
        off = (uint32_t)(row < rows ? row : rows - 1) * R::wrow + 16 * (p - row * R::wn0);
    } else if (p < kH0) {
        const int c = p - 16 * R::wn0, row = c / R::an0;
        off = 0x80000000u | ((uint32_t)row * R::arow + 16 * (c - row * R::an0));
    } else if (p < kH0 + 16 * R::wn1) {
        const int c = p - kH0, row = c / R::wn1;
        off = (uint32_t)(row < rows ? row : rows - 1) * R::wrow + 16 * (R::wc1 + c - row * R::wn1);
    } else {
        const int c = p - kH0 - 16 * R::wn1, row = c / R::an1;
        off = 0x80000000u | ((uint32_t)row * R::arow + 16 * (R::ac1 + c - row * R::an1));
    }
    return off;
}

// Issues a wave's whole run; wsrc / asrc: copy starts of its blocks in the
// tile's first weight row and in activation row 0.
template <class R, int M>
__device__ __forceinline__ void sb_copy(const uint8_t *wsrc, const uint8_t *asrc, uint8_t *base, int lane, int rows) {
#pragma unroll
    for (int i = 0; i < sb_copies<R>(M); ++i) {
        const uint32_t off = sb_chunk<R, M>(64 * i + lane, rows);
        const uint8_t *src = (off >> 31) ? asrc + (off & 0x7fffffffu) : wsrc + off;
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(base + i * 1024), 16, 0, 0);
    }
}

// iq2_xxs, m = 5..8 at k == 4096: 16x16 int8 MFMA tiles of 16 weight rows,
// one super-block per wave, two-half copies. Per sub-block j, lane (row
// l % 16, q = l / 16) holds K positions 8q..8q+7, i.e. grid group q: one grid
// entry and one sign mask gathered from LDS (each a typed 8-byte read), the
// signs applied as (mag ^ neg) + (neg & 1 per byte), one v_mfma_i32_16x16x32_i8
// gives S_j and IS += (2 s_j + 1) * S_j (24-bit multiplies); per super-block
// acc = (0.125 * d * ad) * IS, as the other iq2_xxs GEMVs form it. The
// 66-byte weight block of wave v starts o2 = 2 (v % 8) bytes past a 16-byte
// boundary and is copied as 5 chunks from there; its q8_K block as 17 chunks
// from o = 4 (v % 4) bytes before it (the bsums are not needed). Half 0:
// weight chunks 0..2 (d and sub-blocks 0..3, block bytes 0..33, all below copy
// byte 48) and activation chunks 0..8; half 1: weight chunks 2..4 (chunk 2
// twice, so that sub-blocks 4..7, bytes 34..65, lie in one region) and
// activation chunks 8..16 (bytes 132..259 lie at or past copy byte 128). The
// grid and sign tables are copied into LDS by direct loads issued before the
// run. Where a wave's run is 4 KB or more (m >= 6) each wave copies them into
// the front of its own region and reads only that copy, with no barrier (m = 8:
// 5.05 -> 4.91 us); at m = 5 (3 KB runs, 4.78 against 4.89 us that way) waves
// 0..2 copy one shared set, published by a barrier that waits for it only,
// not for the run, which each wave waits for itself.
typedef uint64_t u64_a4 __attribute__((aligned(4)));  // 8-byte value at a dword-aligned address

__host__ __device__ constexpr bool iq2_sb_private_tables(int m) { return sb_copies<Iq2Run>(m) >= 4; }
__host__ __device__ constexpr int iq2_sb_lds_bytes(int m) {
    return iq2_sb_private_tables(m) ? kKqMfWaves * (kIq2TableBytes + sb_copies<Iq2Run>(m) * 1024)
                                    : kIq2TableBytes + kKqMfWaves * sb_copies<Iq2Run>(m) * 1024;
}

template <int M>
__global__ __launch_bounds__(kKqMfWaves * 64) void gemv_iq2_xxs_mfma_sb_kernel(const uint8_t *__restrict__ w,
                                                                               const uint8_t *__restrict__ a,
                                                                               float *__restrict__ c, int n) {
    static_assert(M >= 1 && M <= 16, "one 16-row tile of activation rows");
    using R = Iq2Run;
    constexpr int nsb = kKqMfWaves;  // k == 4096: one super-block per wave
    constexpr int kH0 = sb_half0<R>(M);
    constexpr int kCopies = sb_copies<R>(M);
    constexpr int kAfterHalf0 = kCopies - (kH0 + 63) / 64;  // instructions issued after those writing half 0
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int n0 = blockIdx.x * 16;
    const int o2 = 2 * (wave & 7), o = 4 * (wave & 3);
    constexpr bool kPrivate = iq2_sb_private_tables(M);
    static_assert(kIq2TableBytes == 3 * 1024, "three 1-KB table pieces");
    // grid magnitudes, then sign masks: the wave's own copy at the front of
    // its region, or one shared copy before all regions
    uint8_t *grid = kPrivate ? lds + wave * (kIq2TableBytes + kCopies * 1024) : lds;
    uint8_t *base = kPrivate ? grid + kIq2TableBytes : lds + kIq2TableBytes + wave * kCopies * 1024;
    // the tables by direct loads as well, issued first (their address is fixed
    // at load time), 1 KB each: every wave its three, or waves 0 and 1 the two
    // halves of the grid and wave 2 the sign masks
    if constexpr (kPrivate) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(&kIq2Tables) + 1024 * i + 16 * lane,
                                             (__attribute__((address_space(3))) void *)(grid + 1024 * i), 16, 0, 0);
    } else if (wave < 3) {
        const uint8_t *tsrc = wave < 2 ? reinterpret_cast<const uint8_t *>(&kIq2Grid) + wave * 1024
                                       : reinterpret_cast<const uint8_t *>(&kIq2Signs);
        __builtin_amdgcn_global_load_lds(tsrc + 16 * lane, (__attribute__((address_space(3))) void *)(grid + wave * 1024),
                                         16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    sb_copy<R, M>(w + ((size_t)n0 * nsb + wave) * kIq2Bytes - o2, a + wave * kQ8KBytes - o, base, lane, n - n0);
    // a shared table piece has landed once at most kCopies loads are
    // outstanding; a private copy, issued before the run, is covered by the
    // run's own first wait
    if constexpr (!kPrivate) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kCopies) : "memory");
    const int li = lane & 15, q = lane >> 4;  // q: the sub-block's group of 8 K positions this lane holds
    const int arow = li < M ? li : M - 1;
    int orow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) orow[r] = 4 * q + r < M ? 4 * q + r : M - 1;
    // weight block byte b sits at copy byte o2 + b: half 0 rows hold copy bytes 0..47, half 1 rows 32..79
    const uint8_t *w0 = base + li * (R::wn0 * 16), *a0 = base + 16 * R::wn0 * 16;
    const uint8_t *w1 = base + kH0 * 16 + li * (R::wn1 * 16) - 16 * R::wc1, *a1 = base + kH0 * 16 + 16 * R::wn1 * 16;
    // activation byte b of row r: half 0 at a0 + 144 r + o + b (b < 144 - o), half 1 at a1 + 144 r + o + b - 128 (b >= 128 - o)
    const uint8_t *ar0 = a0 + arow * (R::an0 * 16) + o, *ar1 = a1 + arow * (R::an1 * 16) + o - R::ac1 * 16;
    const uint32_t sh = (uint32_t)(o2 + 2) & 3u;  // bytes of a sub-block into its first dword
    int is[4] = {0, 0, 0, 0};
    auto sub = [&](const uint8_t *wr, int j, const uint8_t *ar) {
        const uint32_t *p = reinterpret_cast<const uint32_t *>(wr + ((o2 + 2 + 8 * j) & ~3));
        const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
        const uint32_t gidx = __builtin_amdgcn_alignbyte(d1, d0, sh), ss = __builtin_amdgcn_alignbyte(d2, d1, sh);
        // group q of the sub-block: its grid entry and sign mask, and its 8
        // activation bytes (dword-aligned), each read as one typed 8-byte
        // value so that the compiler adds no wait for the copies before it
        const uint64_t mag = *reinterpret_cast<const uint64_t *>(grid + ((gidx >> (8 * q)) & 0xffu) * 8);
        const uint64_t neg = *reinterpret_cast<const uint64_t *>(grid + 256 * 8 + ((ss >> (7 * q)) & 0x7fu) * 8);
        const uint64_t v = (mag ^ neg) + (neg & 0x0101010101010101ull);  // no carry crosses a byte: |mag| >= 8
        const uint64_t y = *reinterpret_cast<const u64_a4 *>(ar + 4 + 32 * j + 8 * q);
        const i32x4 sj = mfma_i8_16x16x32(y, v, (i32x4){0, 0, 0, 0});
        const int scale = 2 * (int)(ss >> 28) + 1;
#pragma unroll
        for (int r = 0; r < 4; ++r) is[r] += __mul24(scale, sj[r]);
    };
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfterHalf0) : "memory");  // half 0 has landed
#pragma unroll
    for (int j = 0; j < 4; ++j) sub(w0, j, ar0);
    const float t0 = 0.125f * fp16_to_f32(*reinterpret_cast<const uint16_t *>(w0 + o2));
    float ad[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ad[r] = *reinterpret_cast<const float *>(a0 + orow[r] * (R::an0 * 16) + o);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 4; j < 8; ++j) sub(w1, j, ar1);
    float acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = (t0 * ad[r]) * (float)is[r];
    __syncthreads();
    float *red = reinterpret_cast<float *>(lds);
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((wave - 1) * 4 + r) * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (wave == 0) {
        for (int v = 1; v < kKqMfWaves; ++v) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] += red[((v - 1) * 4 + r) * 64 + lane];
        }
        const int col = n0 + li;
        if (col < n) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (4 * q + r < M) c[(size_t)(4 * q + r) * n + col] = acc[r];
        }
    }
}

// At kq_tiles_take_k and from m = kq_tiles_min_m up to m = gemv_tiles_max_m:
// 16x16 int8 MFMA tiles of 16 weight rows with one super-block per wave and
// round (round r takes super-block 16 r + wave of every row while it exists,
// so waves can run different numbers of rounds, or none below k = 4096; the
// partial sums stay in registers), the activation rows taken in C = ceil(m / 16)
// chunks of 16. Each wave copies its
// super-block of the tile's 16 weight rows once, decodes them once into
// registers, and then streams the chunks: chunk c's activation blocks arrive in two halves (H0:
// copy chunks 0..8 of each row, d and sub-blocks 0..3; H1: chunks 8..18 or
// 8..16, sub-blocks 4..7 and the bsums), each half into its own LDS buffer,
// which is refilled with chunk c + 1 as soon as the wave has read it: the
// copy of H0(c + 1) runs while H1(c) is multiplied and the copy of H1(c + 1)
// while H0(c + 1) is. Every wait is for the instructions that wrote one
// buffer (loads complete in issue order). Activation rows past m repeat row
// m - 1 (their results are not stored). The copies are run_copy runs
// (device_common.h). q4_K's min term sum_j m_j * bsum_j is one
// v_mfma_f32_16x16x16_f16 per chunk: the bsums (|bsum| <= 16 * 127 < 2048)
// and the 6-bit mins are exact in fp16 and the sums of products exact in
// fp32, so IM equals the integer sum. Measured at 4096 x 4096 against the
// former one-chunk-per-launch kernels that copied each super-block's weight and
// activation bytes together in two halves (us): q4_K m = 5 5.01 / 4.66, m = 8
// 5.20 / 4.66, m = 16 5.71 / 4.88 (m = 4 4.55 against 4.66 for the staged
// kernel); iq2_xxs m = 8 5.53 / 5.61, m = 9 5.85 / 5.78, m = 16 6.27 / 5.98.
constexpr int kChunkWaveBytes = 9 * 1024;  // per wave: weight run, H0, H1 (3 KB each)

// A wave stores its partials as soon as it is done and one barrier suffices
// (as gemv_q4_0_mfma_chunk_kernel): with one chunk into a 16 KB region of
// their own past the wave buffers (against a first barrier and shared
// buffers, q4_K 4096 x 4096, m = 8: 4.46 -> 4.43 us), with more chunks into
// the wave's own buffers (iq2_xxs m = 128: 13.00 -> 12.68 us).
constexpr int kChunkPartialBytes = kKqMfWaves * 1024;
__host__ __device__ constexpr int q4k_chunk_lds_bytes(int c) {
    return kKqMfWaves * kChunkWaveBytes + (c == 1 ? kChunkPartialBytes : 0);
}

template <int C, int kG>
__global__ __launch_bounds__(kKqMfWaves * 64) void gemv_q4_K_mfma_chunk_kernel(const uint8_t *__restrict__ w,
                                                                             const uint8_t *__restrict__ a,
                                                                             float *__restrict__ c, int m, int n,
                                                                             int groups) {
    static_assert(C >= 1 && C <= kMaxGemvChunks, "at most kMaxGemvChunks chunks of 16 activation rows");
    // super-blocks of a row (k == 256 nsb, nsb % 4 == 0): kG when it
    // is fixed at compile time (k = 4096: one round, constant strides), else groups
    const int nsb = kG > 0 ? kG : groups;
    const uint32_t kARow = (uint32_t)nsb * kQ8KBytes;
    constexpr int kH = run_copies<16, 11>();  // instructions per half (H1: 11 columns, H0: 9)
    static_assert(run_copies<16, 9>() == kH && run_copies<16, 9>() * 1024 <= 3072, "3 KB per run");
    static_assert(4 * C * 64 * 4 <= kChunkWaveBytes, "a wave's partials fit its buffers");
    static_assert(q4k_chunk_lds_bytes(C) <= 160 * 1024, "the LDS of one CU");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int n0 = blockIdx.x * 16;
    const int o = 4 * (wave & 3);
    uint8_t *wl = lds + wave * kChunkWaveBytes, *h0 = wl + 3072, *h1 = wl + 6144;
    float acc[C][4];
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[ch][r] = 0.0f;
    // round rnd takes the wave's K slice 16 rnd + wave of every row; the next
    // round's copies start once the last round's buffers have been read
    // this wave's rounds: its super-blocks wave, wave + 16, ... below nsb
    const int my_rounds = (nsb - wave + kKqMfWaves - 1) / kKqMfWaves;
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
        const int sb = kKqMfWaves * rnd + wave;
        const uint8_t *asrc = a + sb * kQ8KBytes - o;  // copy start of the wave's block in activation row 0
        auto copy_h0 = [&](int ch) { copy_run<C, 16, 9>(asrc + (size_t)ch * 16 * kARow, kARow, 0, m - 16 * ch, h0, cl); };
        auto copy_h1 = [&](int ch) { run_copy<16, 11>(asrc + (size_t)ch * 16 * kARow, kARow, 8, m - 16 * ch, h1, cl); };
        copy_run<C, 16, 9>(w + ((size_t)n0 * nsb + sb) * 144, nsb * 144, 0, n - n0, wl, cl);
        copy_h0(0);
        copy_h1(0);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // weights and H0(0)
        // the weight row's decode, once: scales, mins, d, dmin and the nibble operands
        const uint8_t *wr = wl + li * 144;
        const uint32_t *hp = reinterpret_cast<const uint32_t *>(wr);
        const uint4 hd = make_uint4(hp[0], hp[1], hp[2], hp[3]);
        const uint32_t scw[2] = {hd.y & 0x3f3f3f3fu, (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u)};
        const uint32_t mnw[2] = {hd.z & 0x3f3f3f3fu, ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u)};
        uint64_t wv[8];
    #pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t x0 = *reinterpret_cast<const uint32_t *>(wr + 16 + 32 * (j / 2) + 4 * q);
            const uint32_t x1 = *reinterpret_cast<const uint32_t *>(wr + 32 + 32 * (j / 2) + 4 * q);
            const uint32_t v0 = (j & 1 ? x0 >> 4 : x0) & 0x0f0f0f0fu, v1 = (j & 1 ? x1 >> 4 : x1) & 0x0f0f0f0fu;
            wv[j] = (uint64_t)v0 | ((uint64_t)v1 << 32);
        }
        const uint32_t mp = (q & 2 ? mnw[1] : mnw[0]) >> (16 * (q & 1));
        const _Float16 m0 = (_Float16)(int)(mp & 0xffu), m1 = (_Float16)(int)((mp >> 8) & 0xffu);
        const f16x4 mm = {m0, m0, m1, m1};
        const float d = fp16_to_f32(hd.x & 0xffffu), dmin = fp16_to_f32(hd.x >> 16);
        // activation byte b of chunk row r: H0 at h0 + 144 r + o + b, H1 at h1 + 176 r + o + b - 128
        const uint8_t *a0 = h0 + li * 144 + o + 4 + 4 * q, *a1 = h1 + li * 176 + o - 128 + 4 + 4 * q;
    #pragma unroll
        for (int ch = 0; ch < C; ++ch) {
            if (ch > 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // H0(ch)
            int is[4] = {0, 0, 0, 0};
            auto sub = [&](int j, const uint8_t *ay) {
                const uint32_t y0 = *reinterpret_cast<const uint32_t *>(ay + 32 * j);
                const uint32_t y1 = *reinterpret_cast<const uint32_t *>(ay + 32 * j + 16);
                const i32x4 sj = mfma_i8_16x16x32((uint64_t)y0 | ((uint64_t)y1 << 32), wv[j], (i32x4){0, 0, 0, 0});
                const int sc = (int)((scw[j / 4] >> (8 * (j % 4))) & 0xffu);
    #pragma unroll
                for (int r = 0; r < 4; ++r) is[r] += __mul24(sc, sj[r]);
            };
    #pragma unroll
            for (int j = 0; j < 4; ++j) sub(j, a0);
            float ad[4];
    #pragma unroll
            for (int r = 0; r < 4; ++r) ad[r] = *reinterpret_cast<const float *>(h0 + (4 * q + r) * 144 + o);
            if (ch + 1 < C) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // H0 read: refill it
                copy_h0(ch + 1);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // H1(ch)
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
    #pragma unroll
            for (int j = 4; j < 8; ++j) sub(j, a1);
            // IM: A = bsums 4q..4q+3 of the lane's activation row, B = the mins (mm)
            const uint32_t b01 = *reinterpret_cast<const uint32_t *>(a1 - 4 - 4 * q + 260 + 8 * q);
            const uint32_t b23 = *reinterpret_cast<const uint32_t *>(a1 - 4 - 4 * q + 264 + 8 * q);
            const f16x4 bs = {(_Float16)(short)(b01 & 0xffffu), (_Float16)(short)(b01 >> 16),
                              (_Float16)(short)(b23 & 0xffffu), (_Float16)(short)(b23 >> 16)};
            const f32x4 im = __builtin_amdgcn_mfma_f32_16x16x16f16(bs, mm, (f32x4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    #pragma unroll
            for (int r = 0; r < 4; ++r) acc[ch][r] += ad[r] * fmaf(-dmin, im[r], d * (float)is[r]);
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
    float *red = reinterpret_cast<float *>(lds + (C == 1 ? kKqMfWaves * kChunkWaveBytes : 0));
    constexpr int kStride = (C == 1 ? 1024 : kChunkWaveBytes) / 4;
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * kStride + (ch * 4 + r) * 64 + lane] = acc[ch][r];
    __syncthreads();
    const int col = n0 + li;
    for (int g = wave; g < 4 * C; g += kKqMfWaves) {
        float s = red[g * 64 + lane];
        for (int v = 1; v < kKqMfWaves; ++v) s += red[v * kStride + g * 64 + lane];
        const int row = 16 * (g / 4) + 4 * q + g % 4;
        if (col < n && row < m) store_through(&c[(size_t)row * n + col], s);
    }
}

// iq2_xxs, from k = 4096 at k % 2048 == 0: as gemv_q4_K_mfma_chunk_kernel, with the
// weight decode of gemv_iq2_xxs_mfma_sb_kernel done once per wave (5 weight
// columns per row, H1 = activation chunks 8..16). Every wave copies the grid
// and sign tables into its own LDS region before everything else and reads
// only that copy, so no wave waits at a workgroup barrier for another's
// table (against one shared copy behind a barrier, 4096 x 4096: M = 16
// 5.20 -> 4.70 us, M = 32 6.04 -> 5.54, M = 128 13.95 -> 13.11).
// To fit 16 such regions the runs are copied without pad (run_copy_exact):
// per wave the tables (3 KB), the weight run (1280 B) and H0, H1 (2304 B each).
constexpr int kIq2ChunkRunW = 16 * 5 * 16, kIq2ChunkRunH = 16 * 9 * 16;
constexpr int kIq2ChunkWaveBytes = kIq2TableBytes + kIq2ChunkRunW + 2 * kIq2ChunkRunH;  // 8960

__host__ __device__ constexpr int iq2_chunk_lds_bytes(int c) {
    return kKqMfWaves * kIq2ChunkWaveBytes + (c == 1 ? kChunkPartialBytes : 0);
}

template <int C, int kG>
__global__ __launch_bounds__(kKqMfWaves * 64) void gemv_iq2_xxs_mfma_chunk_kernel(const uint8_t *__restrict__ w,
                                                                                const uint8_t *__restrict__ a,
                                                                                float *__restrict__ c, int m, int n,
                                                                                int groups) {
    static_assert(C >= 1 && C <= kMaxGemvChunks, "at most kMaxGemvChunks chunks of 16 activation rows");
    // super-blocks of a row (k == 256 nsb, nsb % 8 == 0): kG when it
    // is fixed at compile time (k = 4096: one round, constant strides), else groups
    const int nsb = kG > 0 ? kG : groups;
    const uint32_t kARow = (uint32_t)nsb * kQ8KBytes;
    constexpr int kH = run_copies<16, 9>();  // instructions per copy (run_copy_exact issues as many)
    static_assert(kIq2ChunkRunH == 16 * 9 * 16 && kIq2ChunkRunW == 16 * 5 * 16, "run sizes");
    static_assert(4 * C * 64 * 4 <= kIq2ChunkWaveBytes, "a wave's partials fit its buffers");
    static_assert(iq2_chunk_lds_bytes(C) <= 160 * 1024, "the LDS of one CU");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int n0 = blockIdx.x * 16;
    const int o2 = 2 * (wave & 7), o = 4 * (wave & 3);
    uint8_t *grid = lds + wave * kIq2ChunkWaveBytes;  // grid magnitudes, then sign masks
    uint8_t *wl = grid + kIq2TableBytes, *h0 = wl + kIq2ChunkRunW, *h1 = h0 + kIq2ChunkRunH;
    static_assert(kIq2TableBytes == 3 * 1024, "three 1-KB table pieces");
    // the table's address is fixed at load time: its copies go out first
#pragma unroll
    for (int i = 0; i < 3; ++i)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(&kIq2Tables) + 1024 * i + 16 * lane,
                                         (__attribute__((address_space(3))) void *)(grid + 1024 * i), 16, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    float acc[C][4];
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[ch][r] = 0.0f;
    // round rnd takes the wave's K slice 16 rnd + wave of every row; the next
    // round's copies start once the last round's buffers have been read
    // this wave's rounds: its super-blocks wave, wave + 16, ... below nsb
    const int my_rounds = (nsb - wave + kKqMfWaves - 1) / kKqMfWaves;
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
        const int sb = kKqMfWaves * rnd + wave;
        const uint8_t *asrc = a + sb * kQ8KBytes - o;
        auto copy_h0 = [&](int ch) {
            run_copy_exact<16, 9>(asrc + (size_t)ch * 16 * kARow, kARow, 0, m - 16 * ch, h0, cl);
        };
        auto copy_h1 = [&](int ch) {
            run_copy_exact<16, 9>(asrc + (size_t)ch * 16 * kARow, kARow, 8, m - 16 * ch, h1, cl);
        };
        run_copy_exact<16, 5>(w + ((size_t)n0 * nsb + sb) * kIq2Bytes - o2, nsb * kIq2Bytes, 0, n - n0, wl, cl);
        copy_h0(0);
        copy_h1(0);
        // weights and H0(0) (and, issued before them, the table copies)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");
        // the weight row's decode, once: group q of every sub-block, its scale, d
        const uint8_t *wr = wl + li * 80;  // weight block byte b at copy byte o2 + b
        const uint32_t sh = (uint32_t)(o2 + 2) & 3u;
        uint64_t wv[8];
        int scale[8];
    #pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t *p = reinterpret_cast<const uint32_t *>(wr + ((o2 + 2 + 8 * j) & ~3));
            const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
            const uint32_t gidx = __builtin_amdgcn_alignbyte(d1, d0, sh), ss = __builtin_amdgcn_alignbyte(d2, d1, sh);
            const uint64_t mag = *reinterpret_cast<const uint64_t *>(grid + ((gidx >> (8 * q)) & 0xffu) * 8);
            const uint64_t neg = *reinterpret_cast<const uint64_t *>(grid + 256 * 8 + ((ss >> (7 * q)) & 0x7fu) * 8);
            wv[j] = (mag ^ neg) + (neg & 0x0101010101010101ull);  // no carry crosses a byte: |mag| >= 8
            scale[j] = 2 * (int)(ss >> 28) + 1;
        }
        const float t0 = 0.125f * fp16_to_f32(*reinterpret_cast<const uint16_t *>(wr + o2));
        // activation bytes 4 + 32 j + 8q (+ 4) of chunk row li: H0 at h0 + 144 li + o + b, H1 at h1 + 144 li + o + b - 128
        const uint8_t *a0 = h0 + li * 144 + o + 4 + 8 * q, *a1 = h1 + li * 144 + o - 128 + 4 + 8 * q;
    #pragma unroll
        for (int ch = 0; ch < C; ++ch) {
            if (ch > 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // H0(ch)
            int is[4] = {0, 0, 0, 0};
            auto sub = [&](int j, const uint8_t *ay) {
                // one typed 8-byte read: the compiler then adds no wait for every outstanding copy before it
                const uint64_t y = *reinterpret_cast<const u64_a4 *>(ay + 32 * j);
                const i32x4 sj = mfma_i8_16x16x32(y, wv[j], (i32x4){0, 0, 0, 0});
    #pragma unroll
                for (int r = 0; r < 4; ++r) is[r] += __mul24(scale[j], sj[r]);
            };
    #pragma unroll
            for (int j = 0; j < 4; ++j) sub(j, a0);
            float ad[4];
    #pragma unroll
            for (int r = 0; r < 4; ++r) ad[r] = *reinterpret_cast<const float *>(h0 + (4 * q + r) * 144 + o);
            if (ch + 1 < C) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // H0 read: refill it
                copy_h0(ch + 1);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kH) : "memory");  // H1(ch)
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
    #pragma unroll
            for (int j = 4; j < 8; ++j) sub(j, a1);
    #pragma unroll
            for (int r = 0; r < 4; ++r) acc[ch][r] += (t0 * ad[r]) * (float)is[r];
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
    float *red = reinterpret_cast<float *>(lds + (C == 1 ? kKqMfWaves * kIq2ChunkWaveBytes : 0));
    constexpr int kStride = (C == 1 ? 1024 : kIq2ChunkWaveBytes) / 4;
    // from two chunks the partials go where the table copy lands, for which a
    // wave with no super-block (nsb < 16) has not waited; the others have
    // waited for everything
    if constexpr (C > 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * kStride + (ch * 4 + r) * 64 + lane] = acc[ch][r];
    __syncthreads();
    const int col = n0 + li;
    for (int g = wave; g < 4 * C; g += kKqMfWaves) {
        float s = red[g * 64 + lane];
        for (int v = 1; v < kKqMfWaves; ++v) s += red[v * kStride + g * 64 + lane];
        const int row = 16 * (g / 4) + 4 * q + g % 4;
        if (col < n && row < m) store_through(&c[(size_t)row * n + col], s);
    }
}

// One launch of the q4_K or iq2_xxs chunk kernel with C chunks over nsb
// super-blocks, the k = 4096 form (16 super-blocks, one round) where it applies.
template <int C>
void launch_kq_chunk(bool q4k, const uint8_t *w, const uint8_t *a, float *c, int m, int n, int nsb,
                     hipStream_t stream) {
    const dim3 grid((unsigned)((n + 15) / 16)), block(kKqMfWaves * 64);
    const size_t lds = q4k ? (size_t)q4k_chunk_lds_bytes(C) : (size_t)iq2_chunk_lds_bytes(C);
    if (q4k && nsb == kKqMfWaves)
        hipLaunchKernelGGL((gemv_q4_K_mfma_chunk_kernel<C, kKqMfWaves>), grid, block, lds, stream, w, a, c, m, n, nsb);
    else if (q4k)
        hipLaunchKernelGGL((gemv_q4_K_mfma_chunk_kernel<C, 0>), grid, block, lds, stream, w, a, c, m, n, nsb);
    else if (nsb == kKqMfWaves)
        hipLaunchKernelGGL((gemv_iq2_xxs_mfma_chunk_kernel<C, kKqMfWaves>), grid, block, lds, stream, w, a, c, m, n,
                           nsb);
    else
        hipLaunchKernelGGL((gemv_iq2_xxs_mfma_chunk_kernel<C, 0>), grid, block, lds, stream, w, a, c, m, n, nsb);
}

// k the chunked MFMA tile kernels take: every row's blocks at the same offset
// from a 16-byte boundary, with the last block's copy ending at the row's end
// (q4_K: k % 1024 == 0, the q8_K blocks' offset set by the block index mod 4;
// iq2_xxs: k % 2048 == 0, its 66-byte weight blocks' offset by the index mod
// 8). Below k = 4096 the waves past the last super-block idle.
bool kq_tiles_take_k(int type, int64_t k) {
    const int64_t unit = type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K ? 1024 : 2048;
    return k % unit == 0 && k >= unit;
}

// Smallest m from which the one-chunk tile runs, measured at n = 4096 against
// the staged kernels (us, tile / staged): q4_K k = 1024 m = 3 3.17 / 3.51;
// k = 2048 m = 4 3.63 / 3.93 (m = 3 3.64 / 3.70); k = 3072 m = 4 3.94 / 4.14
// (m = 3 3.95 / 3.94); k = 4096 m = 5 4.66 / 5.12 (m = 4 4.66 / 4.55); k = 8192
// m = 5 7.83 / 8.25. iq2_xxs k = 2048 m = 5 4.03 / 4.13 (m = 4 4.05 / 3.70);
// k = 4096 from m = 9, m = 5..8 taking the two-half-copy kernel (4096 x 4096
// against the staged kernel, us: m = 4 5.23 / 5.08, m = 5 5.34 / 5.91, m = 8
// 5.56 / 6.58); above 4096 m = 5 (k = 8192 m = 5 8.29 / 9.46, m = 12 8.87 /
// 16.72; k = 14336 m = 8 12.54 / 18.98).
int kq_tiles_min_m(int type, int64_t k) {
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) return k == 4096 ? 9 : 5;
    if (k <= 1024) return 3;
    return k < 4096 ? 4 : 5;
}

template <int M>
hipError_t launch_kq_gemv(int type, const void *w, const void *a, float *c, int64_t n, int64_t k,
                          hipStream_t stream) {
    const auto *wp = static_cast<const uint8_t *>(w);
    const auto *ap = static_cast<const uint8_t *>(a);
    const int64_t nsb = k / 256;
    if constexpr (M >= 3) {
        // one chunk of the chunked kernel from m = kq_tiles_min_m(type, k)
        if (M >= kq_tiles_min_m(type, k) && kq_tiles_take_k(type, k)) {
            launch_kq_chunk<1>(type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K, wp, ap, c, M, (int)n, (int)nsb, stream);
            return hipGetLastError();
        }
    }
    if constexpr (M >= 5) {
        // iq2_xxs m = 5..8 at k = 4096: the two-half-copy kernel
        if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K && k == 4096) {
            const dim3 tiles((unsigned)((n + 15) / 16)), block(kKqMfWaves * 64);
            hipLaunchKernelGGL(gemv_iq2_xxs_mfma_sb_kernel<M>, tiles, block, (size_t)iq2_sb_lds_bytes(M), stream, wp,
                               ap, c, (int)n);
            return hipGetLastError();
        }
    }
    if constexpr (M >= 2) {
        if (kq_staged_lds_bytes(M, nsb) <= 160 * 1024) {
            const dim3 sgrid((unsigned)((n + kStagedThreads / 64 - 1) / (kStagedThreads / 64)));
            const size_t lds = (size_t)kq_staged_lds_bytes(M, nsb);
            if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K)
                hipLaunchKernelGGL(gemv_q4_K_staged_kernel<M>, sgrid, dim3(kStagedThreads), lds, stream, wp, ap, c,
                                   (int)n, (int)nsb);
            else
                hipLaunchKernelGGL(gemv_iq2_xxs_staged_kernel<M>, sgrid, dim3(kStagedThreads), lds, stream, wp, ap, c,
                                   (int)n, (int)nsb);
            return hipGetLastError();
        }
    }
    if constexpr (M <= 8) {
        // activations read from global memory (m == 1, or rows too long to stage)
        const dim3 grid((unsigned)((n + kThreads / 64 - 1) / (kThreads / 64)));
        // q4_K m == 1: activation row in LDS (3.81 against 3.99 us at 4096 x 4096;
        // iq2_xxs, whose decode rather than its activation reads sets its time,
        // measured no change and keeps the global reads)
        if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K && M == 1 && nsb * kQ8KBytes <= 65536)
            hipLaunchKernelGGL((gemv_q4_K_kernel<1, true>), dim3((unsigned)((n + 15) / 16)), dim3(kM1LdsThreads),
                               (size_t)nsb * kQ8KBytes, stream, wp, ap, c, (int)n, (int)nsb);
        else if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K)
            hipLaunchKernelGGL(gemv_q4_K_kernel<M>, grid, dim3(kThreads), 0, stream, wp, ap, c, (int)n,
                               (int)(k / 256));
        else
            hipLaunchKernelGGL(gemv_iq2_xxs_kernel<M>, grid, dim3(kThreads), 0, stream, wp, ap, c, (int)n,
                               (int)(k / 256));
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Fused quantize + GEMV at m == 1 while the q8_K row (and for iq2_xxs the
// tables) fit in 64 KB of LDS. Measured at 4096 x 4096, compute() fused
// against quantize + GEMV: q4_K 4.34 vs 5.7 us, iq2_xxs 5.02 vs 6.1 us.
bool kquant_fused_gemv_fits(int type, int64_t m, int64_t k) {
    if (m != 1 || k % 256 != 0 || k <= 0) return false;
    const int64_t act = (k / 256) * kQ8KBytes;
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) return act <= 65536;
    return type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K && act + kIq2TableBytes <= 65536;
}

hipError_t launch_kquant_fused_gemv(int type, const void *w, const float *x, float *c, int64_t n, int64_t k,
                                    hipStream_t stream) {
    const auto *wp = static_cast<const uint8_t *>(w);
    const int nsb = (int)(k / 256);
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) {
        hipLaunchKernelGGL((gemv_q4_K_kernel<1, true, true>), dim3((unsigned)((n + 15) / 16)), dim3(kM1LdsThreads),
                           (size_t)nsb * kQ8KBytes, stream, wp, reinterpret_cast<const uint8_t *>(x), c, (int)n, nsb);
        return hipGetLastError();
    }
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) {
        // 16 rows per workgroup: 5.02 us at 4096 x 4096 against 7.42 with 4
        // (each workgroup quantizes the whole row), 6.0 unfused
        constexpr int kWaves = 16;
        hipLaunchKernelGGL(gemv_iq2_xxs_fused_kernel<kWaves>, dim3((unsigned)((n + kWaves - 1) / kWaves)),
                           dim3(kWaves * 64), (size_t)(kIq2TableBytes + nsb * kQ8KBytes), stream, wp, x, c, (int)n,
                           nsb);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

bool kquant_gemv_staged_fits(int64_t m, int64_t k) {
    return m >= 2 && m <= 16 && k % 256 == 0 && kq_staged_lds_bytes(m, k / 256) <= 160 * 1024;
}

bool kquant_gemv_chunked_fits(int type, int64_t m, int64_t k) {
    return m >= 9 && m <= gemv_tiles_max_m(k) && kq_tiles_take_k(type, k);
}

hipError_t launch_kquant_gemv(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                              hipStream_t stream) {
    if (type != PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K && type != PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K)
        return hipErrorInvalidValue;
    switch (m) {
    case 1: return launch_kq_gemv<1>(type, w, a, c, n, k, stream);
    case 2: return launch_kq_gemv<2>(type, w, a, c, n, k, stream);
    case 3: return launch_kq_gemv<3>(type, w, a, c, n, k, stream);
    case 4: return launch_kq_gemv<4>(type, w, a, c, n, k, stream);
    case 5: return launch_kq_gemv<5>(type, w, a, c, n, k, stream);
    case 6: return launch_kq_gemv<6>(type, w, a, c, n, k, stream);
    case 7: return launch_kq_gemv<7>(type, w, a, c, n, k, stream);
    case 8: return launch_kq_gemv<8>(type, w, a, c, n, k, stream);
    case 9: return launch_kq_gemv<9>(type, w, a, c, n, k, stream);
    case 10: return launch_kq_gemv<10>(type, w, a, c, n, k, stream);
    case 11: return launch_kq_gemv<11>(type, w, a, c, n, k, stream);
    case 12: return launch_kq_gemv<12>(type, w, a, c, n, k, stream);
    case 13: return launch_kq_gemv<13>(type, w, a, c, n, k, stream);
    case 14: return launch_kq_gemv<14>(type, w, a, c, n, k, stream);
    case 15: return launch_kq_gemv<15>(type, w, a, c, n, k, stream);
    case 16: return launch_kq_gemv<16>(type, w, a, c, n, k, stream);
    default: break;
    }
    if (!kquant_gemv_chunked_fits(type, m, k)) return hipErrorInvalidValue;
    const auto *wp = static_cast<const uint8_t *>(w);
    const auto *ap = static_cast<const uint8_t *>(a);
    const bool q4k = type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K;
    const int ng = (int)(k / 256);
#define PFNG_CHUNK_CASE(C)                                                                                      \
    case C:                                                                                                    \
        launch_kq_chunk<C>(q4k, wp, ap, c, (int)m, (int)n, ng, stream);                                        \
        return hipGetLastError();
    switch ((m + 15) / 16) {
        PFNG_CHUNK_CASE(2)
        PFNG_CHUNK_CASE(3)
        PFNG_CHUNK_CASE(4)
        PFNG_CHUNK_CASE(5)
        PFNG_CHUNK_CASE(6)
        PFNG_CHUNK_CASE(7)
        PFNG_CHUNK_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef PFNG_CHUNK_CASE
}

}  // namespace pfng
