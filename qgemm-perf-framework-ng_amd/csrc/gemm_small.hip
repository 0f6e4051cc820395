// q4_0 x q8_0 int8-MFMA GEMM for small problems whose whole K range fits in
// LDS (e.g. 480x1536x1536): one workgroup per CU-sized output tile of
// 32 x 32*TN, the tile's operands copied into LDS once, K split over the
// waves.
//
// Copy: the tile's 32 activation rows and 32*TN weight rows are each one
// contiguous run of memory (row-major blocks, all of K), copied with 16-byte
// direct-to-LDS buffer loads, 1 KB per instruction and no vector ALU work per
// copy: L2 -> LDS moves long runs several times faster than row-strided
// pieces (measured: 68-byte row pieces by 4-byte lanes ~18 B/clk/CU, long
// 16-byte runs ~73 B/clk/CU; a phase-major layout with 144- and 272-byte row
// pieces of 16-byte lanes cost 1.1 us more at 480x1536x1536). Rows are laid
// out in LDS as in memory, each padded to an odd number of 16-byte chunks, and
// row r's data starts s(r) = (r % 32) / 8 dwords into its first chunk (the
// copy fetches each chunk 4 s(r) bytes early). The fragment reads are dwords,
// 32 lanes on 32 rows; the LDS serves them 32 lanes at a time over 32 banks.
// With the row stride an odd number of chunks (4 mod 8 dwords) rows r = 0..7
// land on distinct multiples of 4 and the shift fills the banks in between,
// so every read is conflict-free (without the shift four lanes shared each
// bank: 8.45 against 7.38 us at 480x1536x1536).
// Compute: wave w takes column tile w % TN and block pairs
// [(w / TN)*PPW, (w / TN + 1)*PPW) of its rows (K slice w / TN of WS). Per
// block: S16 = v_mfma_i32_32x32x32_i8 (exact 16*S_b) on the raw bytes (the
// first block of a pair realigned by two bytes, nibbles widened to 16*(q-8)
// int8), P = da (x) dw by v_mfma_f32_32x32x8_f16 on one-hot fp16 operands
// (exact), acc = fma(S16, P, acc). The WS partial tiles of a column tile are
// then added through LDS in slice order (results do not depend on timing);
// C = acc / 16.
//
// Integer parts are exact; the fp32 result differs from the reference's
// block-sequential sum (llama_reference.cpp:134-146) only by reassociation.
#include "device_common.h"
#include "kernels.h"

namespace pfng {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kBufferWord3 = 0x00020000u;  // raw buffer resource, gfx9 family

// One 16-byte direct-to-LDS buffer load per lane (64 lanes: 1 KB at dst). A
// plain function: inside a kernel template the 16-byte form of the builtin
// makes the host pass drop the kernel's launch stub.
__device__ __forceinline__ void copy16_to_lds(__amdgpu_buffer_rsrc_t r, uint8_t *dst, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)dst, 16, voffset, 0, 0, 0);
}

template <int TN, int WS, int NB>
struct WtConfig {
    static constexpr int WK = WS * TN;  // waves
    static constexpr int kThreads = 64 * WK;
    static_assert(NB % 8 == 0, "a row is whole 16-byte chunks (8 blocks)");
    static_assert((NB / 2) % WS == 0, "every wave takes whole block pairs");
    static constexpr int kPPW = NB / 2 / WS;  // block pairs per wave
    // 16-byte chunks of a row: data, and the LDS row: at least one more (the
    // shifted row's end), an odd number
    static constexpr int kDataA = NB * 34 / 16, kDataW = NB * 18 / 16;
    static constexpr int kChunksA = (kDataA + 1) | 1, kChunksW = (kDataW + 1) | 1;
    static constexpr int kRowsW = 32 * TN;
    static constexpr int kCopiesA = (32 * kChunksA + 63) / 64;  // 64 chunks per copy instruction
    static constexpr int kCopiesW = (kRowsW * kChunksW + 63) / 64;
    static constexpr int kCopiesPerWave = (kCopiesA + kCopiesW + WK - 1) / WK;
    static constexpr int kBytesA = kCopiesA * 1024, kBytesW = kCopiesW * 1024;
    static constexpr int kGroupBytes = WK * 64 * 16;  // one float4 register group of every wave
    static_assert(kBytesA + kBytesW <= 160 * 1024, "tile must fit in LDS");
    static_assert(4 * kGroupBytes <= kBytesW, "partial tiles fit in the weight buffer");
};

// dword shift of tile row r inside its LDS row
__device__ __forceinline__ int row_skew(int r) { return (r & 31) >> 3; }

// Byte offset in memory (from the tile's first row) of this lane's chunk in
// copy instruction j of a region of `rows` LDS rows of C chunks (D of data,
// C > D): LDS chunk (r, col) holds the row's bytes [16 col - 4 s(r), +16), so
// the last chunk carries the end of the shifted row. Lanes past the region
// repeat its last chunk, rows past `rows_valid` repeat the last valid row
// (shifted like the row whose place they fill), offsets before the tile are
// clamped to it, and offsets past the buffer's end read zeros (the buffer
// resource is bounded).
// Rows RB bytes apart in memory (the q4_0 rows are whole chunks, RB = 16 D);
// kSkew false: no shift (rows read as 16-byte fragments).
template <int C, int RB, bool kSkew>
__device__ __forceinline__ uint32_t chunk_source_rb(int j, int lane, int rows, int rows_valid) {
    static_assert(16 * C >= RB + (kSkew ? 12 : 0), "room for the (shifted) row");
    int i = 64 * j + lane;
    if (i >= rows * C) i = rows * C - 1;
    const int r = i / C;
    const int col = i - r * C;
    const int rr = r < rows_valid ? r : rows_valid - 1;
    const int off = rr * RB + col * 16 - (kSkew ? 4 * row_skew(r) : 0);
    return (uint32_t)(off > 0 ? off : 0);
}
template <int C, int D>
__device__ __forceinline__ uint32_t chunk_source(int j, int lane, int rows, int rows_valid) {
    static_assert(C > D, "room for the shifted row");
    return chunk_source_rb<C, D * 16, true>(j, lane, rows, rows_valid);
}

// This wave's copy instructions (activation rows into bufa, weight rows
// into bufw), dealt round-robin over the waves.
template <class Cfg>
__device__ __forceinline__ void copy_tile(uint8_t *bufa, uint8_t *bufw, __amdgpu_buffer_rsrc_t ra,
                                          __amdgpu_buffer_rsrc_t rw, int wave, int lane, int rows_a, int rows_w) {
    constexpr int kTotal = Cfg::kCopiesA + Cfg::kCopiesW;
#pragma unroll
    for (int i = 0; i < Cfg::kCopiesPerWave; ++i) {
        int j = wave + i * Cfg::WK;
        if (j >= kTotal) j = kTotal - 1;
        if (j < Cfg::kCopiesA)
            copy16_to_lds(ra, bufa + j * 1024,
                          chunk_source<Cfg::kChunksA, Cfg::kDataA>(j, lane, 32, rows_a));
        else
            copy16_to_lds(rw, bufw + (j - Cfg::kCopiesA) * 1024,
                          chunk_source<Cfg::kChunksW, Cfg::kDataW>(j - Cfg::kCopiesA, lane, Cfg::kRowsW, rows_w));
    }
}

// The wave's block pairs against its column tile.
template <class Cfg, bool kIsums>
__device__ __forceinline__ void compute_slice(const uint8_t *bufa, const uint8_t *bufw, int tile, int slice, int lane,
                                              f32x16 &acc, int32_t *isums, int m, int n, int nb, int m0, int n0) {
    const int li = lane & 31, h = lane >> 5;
    const uint32_t keep = h ? 0u : 0xffffffffu;  // K-half 1 lanes feed zeros to the scale products
    const uint32_t *arow = reinterpret_cast<const uint32_t *>(bufa) + li * Cfg::kChunksA * 4 + row_skew(li);
    const uint32_t *wrow = reinterpret_cast<const uint32_t *>(bufw) + (tile * 32 + li) * Cfg::kChunksW * 4 + row_skew(li);
#pragma unroll
    for (int pp = 0; pp < Cfg::kPPW; ++pp) {
        const int lp = slice * Cfg::kPPW + pp;  // pair within the row
        const uint32_t *sa = arow + lp * 17, *sw = wrow + lp * 9;
        const uint32_t *ah = sa + 2 * h, *wh = sw + 2 * h;
        // block 0 sits two bytes into its dwords, block 1 is dword-aligned
        const i32x4 a0 = (i32x4){(int)shift2(ah[0], ah[1]), (int)shift2(ah[1], ah[2]), (int)shift2(ah[4], ah[5]),
                                 (int)shift2(ah[5], ah[6])};
        const i32x4 a1 = (i32x4){(int)ah[9], (int)ah[10], (int)ah[13], (int)ah[14]};
        const uint32_t u0 = shift2(wh[0], wh[1]), u1 = shift2(wh[1], wh[2]);
        const uint32_t v0 = wh[5], v1 = wh[6];
        const i32x4 b0 = (i32x4){(int)q4_0_lo16(u0), (int)q4_0_lo16(u1), (int)q4_0_hi16(u0), (int)q4_0_hi16(u1)};
        const i32x4 b1 = (i32x4){(int)q4_0_lo16(v0), (int)q4_0_lo16(v1), (int)q4_0_hi16(v0), (int)q4_0_hi16(v1)};
        const i32x16 s0 = mfma_i8_32x32x32(a0, b0, (i32x16){});
        const i32x16 s1 = mfma_i8_32x32x32(a1, b1, (i32x16){});
        if constexpr (kIsums) {
            const int col = n0 + tile * 32 + li;
            const int blk = 2 * lp;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int row = m0 + mfma_row(lane, q);
                if (row < m && col < n) {
                    int32_t *dst = isums + ((size_t)row * n + col) * nb + blk;
                    dst[0] = s0[q] / 16;
                    dst[1] = s1[q] / 16;
                }
            }
        } else {
            const f16x4 pa =
                __builtin_bit_cast(f16x4, make_uint2(__builtin_amdgcn_perm(sa[8], sa[0], 0x07060100u) & keep, 0u));
            const f16x4 pb0 = __builtin_bit_cast(f16x4, make_uint2(sw[0] & keep & 0xffffu, 0u));
            const f16x4 pb1 = __builtin_bit_cast(f16x4, make_uint2(sw[4] & keep & 0xffff0000u, 0u));
            const f32x16 p0 = mfma_f16_32x32x8(pa, pb0, (f32x16){});
            const f32x16 p1 = mfma_f16_32x32x8(pa, pb1, (f32x16){});
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[q] = __builtin_fmaf((float)s0[q], p0[q], acc[q]);
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[q] = __builtin_fmaf((float)s1[q], p1[q], acc[q]);
        }
    }
}

template <int TN, int WS, int NB, bool kIsums>
__global__ __launch_bounds__(64 * WS * TN) void gemm_q4_0_wt_kernel(const uint8_t *__restrict__ w,
                                                                    const uint8_t *__restrict__ a,
                                                                    float *__restrict__ c,
                                                                    int32_t *__restrict__ isums, int m, int n) {
    using Cfg = WtConfig<TN, WS, NB>;
    __shared__ __align__(16) uint8_t a0[Cfg::kBytesA], w0[Cfg::kBytesW];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const TileOrigin to = xcd_tile(blockIdx.x, (m + 31) / 32, (n + Cfg::kRowsW - 1) / Cfg::kRowsW);
    const int m0 = to.mi * 32, n0 = to.ni * Cfg::kRowsW;
    const int tile = wave % TN, slice = wave / TN;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a + (size_t)m0 * NB * 34), 0, (int)((uint32_t)(m - m0) * NB * 34u), kBufferWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(w + (size_t)n0 * NB * 18), 0, (int)((uint32_t)(n - n0) * NB * 18u), kBufferWord3);
    const int rows_a = m - m0 < 32 ? m - m0 : 32;
    const int rows_w = n - n0 < Cfg::kRowsW ? n - n0 : Cfg::kRowsW;
    copy_tile<Cfg>(a0, w0, ra, rw, wave, lane, rows_a, rows_w);
    // this wave's copies have landed, then every wave's
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    f32x16 acc = (f32x16){};
    compute_slice<Cfg, kIsums>(a0, w0, tile, slice, lane, acc, isums, m, n, NB, m0, n0);

    if constexpr (!kIsums) {
        // A wave's partial tile goes into the weight bytes that only it reads
        // (its column tile's rows, its K slice: 9 kPPW dwords a row; lane l's
        // 16 results, all of weight row l % 32, at dwords 16 (l / 32) + q), so
        // it stores them as soon as it is done and one barrier suffices; then
        // each wave adds one group of one column tile over the K slices in
        // order and stores it (480x1536x1536: 7.18 -> 6.65 us against a first
        // barrier and [group][wave][lane] float4 groups, the same bits).
        static_assert(9 * Cfg::kPPW >= 32, "a K slice's part of a weight row holds two lanes' results");
        auto part = [&](int t, int sl, int l) -> uint32_t * {
            const int r = l & 31;
            return reinterpret_cast<uint32_t *>(w0) + (t * 32 + r) * Cfg::kChunksW * 4 + row_skew(r) +
                   sl * Cfg::kPPW * 9 + (l >> 5) * 16;
        };
        {
            uint32_t *dst = part(tile, slice, lane);
#pragma unroll
            for (int q = 0; q < 16; ++q) dst[q] = __float_as_uint(acc[q]);
        }
        __syncthreads();
        const int li = lane & 31;
        for (int tg = wave; tg < TN * 4; tg += Cfg::WK) {
            const int t = tg % TN, g = tg / TN;
            float r[4];
            const uint32_t *p0 = part(t, 0, lane) + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = __uint_as_float(p0[i]);
#pragma unroll
            for (int sl = 1; sl < WS; ++sl) {
                const uint32_t *p = part(t, sl, lane) + 4 * g;
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] += __uint_as_float(p[i]);
            }
            const int col = n0 + t * 32 + li;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = m0 + mfma_row(lane, 4 * g + i);
                if (row < m && col < n) store_through(&c[(size_t)row * n + col], r[i] * 0.0625f);
            }
        }
    }
}

template <int TN, int WS, int NB, bool kIsums>
hipError_t launch_wt(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n, hipStream_t stream) {
    using Cfg = WtConfig<TN, WS, NB>;
    const dim3 grid((unsigned)(((m + 31) / 32) * ((n + Cfg::kRowsW - 1) / Cfg::kRowsW)));
    hipLaunchKernelGGL((gemm_q4_0_wt_kernel<TN, WS, NB, kIsums>), grid, dim3(Cfg::kThreads), 0, stream,
                       static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, isums, (int)m, (int)n);
    return hipGetLastError();
}

template <int TN, int WS, int NB>
hipError_t launch_wt_any(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n,
                         hipStream_t stream) {
    return isums ? launch_wt<TN, WS, NB, true>(w, a, c, isums, m, n, stream)
                 : launch_wt<TN, WS, NB, false>(w, a, c, isums, m, n, stream);
}

// ---------------------------------------------------------------------------
// q4_K x q8_K with the whole K range in LDS (k = 1024 or 1536, e.g.
// 480x1536x1536): the q4_0 tile's plan for the super-block format. Per 32 x 96
// tile the 32 activation rows (q8_K blocks as in memory, each row shifted by
// s(r) dwords, read as dwords like the q4_0 rows) and the 96 weight rows (q4_K
// blocks as in memory, unshifted: 16-byte aligned, read as 16-byte fragments;
// an odd number of chunks per row keeps rows 0..7 of a fragment read on
// distinct banks) are copied into LDS once; then a table of the activation
// scales, [block][row].
// 12 waves = 4 K slices x 3 column tiles; slice S takes sub-blocks
// [S * 2 NB, (S + 1) * 2 NB) of the row's 8 NB, so a slice ends inside a
// super-block where NB is odd (the q4_K accuracy bound is per element, so a
// super-block's partial sums may be scaled separately). Per super-block part,
// as gemm_kquant.hip's q4_K tiles: sc = 8 h + l, two int8 MFMAs per sub-block on
// the planes q * l and q * h (IS = 8 S_H + S_L), IM = sum_j m_j (bsum_2j +
// bsum_2j+1) by one fp16 MFMA (mins of the sub-blocks outside the part are
// zero), then acc += ad * (d * IS - dmin * IM). The slices' partial tiles are
// added through LDS in slice order.
template <int NB>
struct KtConfig {
    static constexpr int TN = 3, WS = 4, WK = WS * TN, kThreads = 64 * WK;
    static constexpr int kRowA = NB * 292, kRowW = NB * 144;
    static constexpr int kChunksA = ((kRowA + 12 + 15) / 16) | 1;  // shifted by up to 12 bytes
    static constexpr int kChunksW = ((kRowW + 15) / 16) | 1;
    static constexpr int kRowsW = 32 * TN;
    static constexpr int kCopiesA = (32 * kChunksA + 63) / 64;
    static constexpr int kCopiesW = (kRowsW * kChunksW + 63) / 64;
    static constexpr int kCopiesPerWave = (kCopiesA + kCopiesW + WK - 1) / WK;
    static constexpr int kBytesA = kCopiesA * 1024, kBytesW = kCopiesW * 1024;
    static constexpr int kSubs = NB * 8 / WS;  // sub-blocks of one K slice
    static constexpr int kGroupBytes = WK * 64 * 16;
    static_assert(NB * 8 % WS == 0, "K slices of whole sub-blocks");
    static_assert(4 * kGroupBytes <= kBytesW, "partial tiles fit in the weight buffer");
    static_assert(kBytesA + kBytesW + NB * 32 * 4 <= 160 * 1024, "tile must fit in LDS");
};

template <class Cfg>
__device__ __forceinline__ void kt_copy_tile(uint8_t *bufa, uint8_t *bufw, __amdgpu_buffer_rsrc_t ra,
                                             __amdgpu_buffer_rsrc_t rw, int wave, int lane, int rows_a, int rows_w) {
    constexpr int kTotal = Cfg::kCopiesA + Cfg::kCopiesW;
#pragma unroll
    for (int i = 0; i < Cfg::kCopiesPerWave; ++i) {
        int j = wave + i * Cfg::WK;
        if (j >= kTotal) j = kTotal - 1;
        if (j < Cfg::kCopiesA)
            copy16_to_lds(ra, bufa + j * 1024,
                          chunk_source_rb<Cfg::kChunksA, Cfg::kRowA, true>(j, lane, 32, rows_a));
        else
            copy16_to_lds(rw, bufw + (j - Cfg::kCopiesA) * 1024,
                          chunk_source_rb<Cfg::kChunksW, Cfg::kRowW, false>(j - Cfg::kCopiesA, lane, Cfg::kRowsW,
                                                                             rows_w));
    }
}

// Slice S of the wave's column tile into acc.
template <class Cfg, int NB, int S>
__device__ __forceinline__ void kt_compute(const uint8_t *bufa, const uint8_t *bufw, const float *adt, int tile,
                                           int lane, f32x16 &acc) {
    constexpr int s0 = S * Cfg::kSubs, s1 = s0 + Cfg::kSubs;
    const int li = lane & 31, lh = lane >> 5;
    const uint32_t *arow = reinterpret_cast<const uint32_t *>(bufa) + li * Cfg::kChunksA * 4 + row_skew(li);
    const uint8_t *wrow = bufw + (tile * 32 + li) * Cfg::kChunksW * 16;
#pragma unroll
    for (int sb = s0 / 8; sb <= (s1 - 1) / 8; ++sb) {
        const int ja = s0 > 8 * sb ? s0 - 8 * sb : 0, jb = s1 < 8 * sb + 8 ? s1 - 8 * sb : 8;
        const uint4 hd = *reinterpret_cast<const uint4 *>(wrow + sb * 144);
        // the reference's scale and min decode (llama_reference.cpp:116-121)
        // four sub-blocks per word: byte i of sc_lo / mn_lo is sub-block i's,
        // of sc_hi / mn_hi sub-block 4 + i's
        const uint32_t sc_lo = hd.y & 0x3f3f3f3fu, mn_lo = hd.z & 0x3f3f3f3fu;
        const uint32_t sc_hi = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mn_hi = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
        // octal digits l, h of the scales, then one sub-block's digit in both
        // 16-bit halves by a byte permute
        const uint32_t dl_lo = sc_lo & 0x07070707u, dh_lo = (sc_lo >> 3) & 0x07070707u;
        const uint32_t dl_hi = sc_hi & 0x07070707u, dh_hi = (sc_hi >> 3) & 0x07070707u;
        i32x16 sl = {}, sh = {};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j < ja || j >= jb) continue;
            // activation bytes 16 lh .. 16 lh + 15 of sub-block j (dword-aligned)
            const uint32_t *ap = arow + sb * 73 + 1 + 8 * j + 4 * lh;
            const i32x4 av = (i32x4){(int)ap[0], (int)ap[1], (int)ap[2], (int)ap[3]};
            // the nibble bytes of pair j / 2: low nibbles sub-block j even, high odd
            const uint4 wq = *reinterpret_cast<const uint4 *>(wrow + sb * 144 + 16 + 32 * (j / 2) + 16 * lh);
            const uint32_t sh4 = (j & 1) ? 4u : 0u;
            const i32x4 nib = (i32x4){(int)((wq.x >> sh4) & 0x0f0f0f0fu), (int)((wq.y >> sh4) & 0x0f0f0f0fu),
                                      (int)((wq.z >> sh4) & 0x0f0f0f0fu), (int)((wq.w >> sh4) & 0x0f0f0f0fu)};
            const uint32_t sel = 0x0c000c00u | (uint32_t)(j & 3) * 0x00010001u;
            const uint32_t d2l = __builtin_amdgcn_perm(0u, j < 4 ? dl_lo : dl_hi, sel);
            const uint32_t d2h = __builtin_amdgcn_perm(0u, j < 4 ? dh_lo : dh_hi, sel);
            const bool first = j == ja;
            sl = mfma_i8_32x32x32(av, mul_planes(nib, d2l), first ? (i32x16){} : sl);
            sh = mfma_i8_32x32x32(av, mul_planes(nib, d2h), first ? (i32x16){} : sh);
        }
        // IM: lane supplies the bsums 8 lh .. 8 lh + 7 of row li (sub-blocks
        // 4 lh .. 4 lh + 3) and the mins of column li for those sub-blocks,
        // each twice (exact: |bsum| <= 2032 and m <= 63 are fp16 integers);
        // the mins of sub-blocks outside [ja, jb) are zeroed
        const uint32_t *bp = arow + sb * 73 + 65 + 4 * lh;
        uint32_t keep_lo = 0, keep_hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i >= ja && i < jb) keep_lo |= 0xffu << (8 * i);
            if (4 + i >= ja && 4 + i < jb) keep_hi |= 0xffu << (8 * i);
        }
        const uint32_t mins = lh ? (mn_hi & keep_hi) : (mn_lo & keep_lo);
        f16x8 bs, mv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t v = bp[i];
            bs[2 * i] = (_Float16)(int16_t)(v & 0xffffu);
            bs[2 * i + 1] = (_Float16)(int16_t)(v >> 16);
            const _Float16 mm = (_Float16)((mins >> (8 * i)) & 0xffu);
            mv[2 * i] = mm;
            mv[2 * i + 1] = mm;
        }
        const f32x16 im = mfma_f16_32x32x16(bs, mv, (f32x16){});
        const float d = fp16_to_f32(hd[0] & 0xffffu), dmin = fp16_to_f32(hd[0] >> 16);
        // activation scales of the lane's 16 rows: rows 8 g + 4 lh + 0..3
        const float *adp = adt + sb * 32 + 4 * lh;
        f32x4 ad4[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) ad4[g] = *reinterpret_cast<const f32x4 *>(adp + 8 * g);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int is = 8 * sh[q] + sl[q];
            const float x = fmaf(-dmin, im[q], d * (float)is);
            acc[q] = fmaf(ad4[q / 4][q % 4], x, acc[q]);
        }
    }
}

template <int NB>
__global__ __launch_bounds__(KtConfig<NB>::kThreads) void gemm_q4_K_wt_kernel(const uint8_t *__restrict__ w,
                                                                             const uint8_t *__restrict__ a,
                                                                             float *__restrict__ c, int m, int n) {
    using Cfg = KtConfig<NB>;
    __shared__ __align__(16) uint8_t a0[Cfg::kBytesA], w0[Cfg::kBytesW];
    __shared__ __align__(16) float adt[NB * 32];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const TileOrigin to = xcd_tile(blockIdx.x, (m + 31) / 32, (n + Cfg::kRowsW - 1) / Cfg::kRowsW);
    const int m0 = to.mi * 32, n0 = to.ni * Cfg::kRowsW;
    const int tile = wave % Cfg::TN, slice = wave / Cfg::TN;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a + (size_t)m0 * Cfg::kRowA), 0, (int)((uint32_t)(m - m0) * (uint32_t)Cfg::kRowA), kBufferWord3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(w + (size_t)n0 * Cfg::kRowW), 0, (int)((uint32_t)(n - n0) * (uint32_t)Cfg::kRowW), kBufferWord3);
    const int rows_a = m - m0 < 32 ? m - m0 : 32;
    const int rows_w = n - n0 < Cfg::kRowsW ? n - n0 : Cfg::kRowsW;
    kt_copy_tile<Cfg>(a0, w0, ra, rw, wave, lane, rows_a, rows_w);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int t = threadIdx.x; t < NB * 32; t += Cfg::kThreads) {
        const int b = t >> 5, r = t & 31;
        adt[t] = *reinterpret_cast<const float *>(a0 + r * Cfg::kChunksA * 16 + 4 * row_skew(r) + b * 292);
    }
    __syncthreads();
    f32x16 acc = (f32x16){};
    switch (slice) {
    case 0: kt_compute<Cfg, NB, 0>(a0, w0, adt, tile, lane, acc); break;
    case 1: kt_compute<Cfg, NB, 1>(a0, w0, adt, tile, lane, acc); break;
    case 2: kt_compute<Cfg, NB, 2>(a0, w0, adt, tile, lane, acc); break;
    default: kt_compute<Cfg, NB, 3>(a0, w0, adt, tile, lane, acc); break;
    }

    // A wave's partial tile goes into weight bytes that only it reads: the
    // nibble bytes (128, 16-byte aligned) of the first super-block that lies
    // wholly inside its K slice, in its column tile's rows (lane l's 16
    // results, all of weight row l % 32, at byte 16 + 64 (l / 32)). So it
    // stores them as soon as it is done and one barrier suffices; then each
    // wave adds one group of one column tile over the K slices in order and
    // stores it (480x1536x1536: 7.05 -> 6.95 us, the same bits).
    auto part = [&](int t, int sl, int l) -> float4 * {
        constexpr int kSubs = Cfg::kSubs;
        const int sb = (sl * kSubs + 7) / 8;  // first super-block wholly in slice sl
        return reinterpret_cast<float4 *>(w0 + (t * 32 + (l & 31)) * Cfg::kChunksW * 16 + sb * 144 + 16 + 64 * (l >> 5));
    };
    static_assert([] {
        for (int sl = 0; sl < Cfg::WS; ++sl)
            if (((sl * Cfg::kSubs + 7) / 8 + 1) * 8 > (sl + 1) * Cfg::kSubs) return false;
        return true;
    }(), "every K slice holds a whole super-block");
    {
        float4 *dst = part(tile, slice, lane);
#pragma unroll
        for (int g = 0; g < 4; ++g) dst[g] = make_float4(acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]);
    }
    __syncthreads();
    const int li = lane & 31;
    for (int tg = wave; tg < Cfg::TN * 4; tg += Cfg::WK) {
        const int t = tg % Cfg::TN, g = tg / Cfg::TN;
        float4 s = part(t, 0, lane)[g];
#pragma unroll
        for (int sl = 1; sl < Cfg::WS; ++sl) {
            const float4 v = part(t, sl, lane)[g];
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        const int col = n0 + t * 32 + li;
        const float r[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m0 + mfma_row(lane, 4 * g + i);
            if (row < m && col < n) store_through(&c[(size_t)row * n + col], r[i]);
        }
    }
}

template <int NB>
hipError_t launch_kt(const void *w, const void *a, float *c, int64_t m, int64_t n, hipStream_t stream) {
    using Cfg = KtConfig<NB>;
    const dim3 grid((unsigned)(((m + 31) / 32) * ((n + Cfg::kRowsW - 1) / Cfg::kRowsW)));
    hipLaunchKernelGGL((gemm_q4_K_wt_kernel<NB>), grid, dim3(Cfg::kThreads), 0, stream,
                       static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, (int)m, (int)n);
    return hipGetLastError();
}

}  // namespace

bool q4_0_small_supported(int64_t k) { return k == 1024 || k == 1536; }

bool q4_K_small_supported(int64_t k) { return k == 1024 || k == 1536; }

hipError_t launch_q4_K_small(const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                             hipStream_t stream) {
    // 32 x 96 tiles, 12 waves: 4 K slices x 3 column tiles
    if (k == 1536) return launch_kt<6>(w, a, c, m, n, stream);
    if (k == 1024) return launch_kt<4>(w, a, c, m, n, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_q4_0_small(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n,
                             int64_t k, hipStream_t stream) {
    // 32 x 96 tiles, 12 waves: 4 K slices x 3 column tiles
    if (k == 1536) return launch_wt_any<3, 4, 48>(w, a, c, isums, m, n, stream);
    if (k == 1024) return launch_wt_any<3, 4, 32>(w, a, c, isums, m, n, stream);
    return hipErrorInvalidValue;
}

}  // namespace pfng
