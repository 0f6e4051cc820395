// int8-MFMA GEMM for the 256-element super-block formats against q8_K
// activations: q4_K (llama_reference.cpp:113-132) and iq2_xxs
// (llama_reference.cpp:148-161 with kernels/common/iq2_xxs.h:29-41).
//
// Both formats carry a small integer scale per 32-element sub-block j and an
// fp16 scale per super-block, so each super-block reduces to exact int32 sums
// before any floating-point work:
//   q4_K:    IS = sum_j sc_j * S_j,  IM = sum_j m_j * (bsum_2j + bsum_2j+1)
//            C += ad * (d * IS - dmin * IM)
//   iq2_xxs: IS = sum_j (2 s_j + 1) * S_j
//            C += (0.125 * d * ad) * IS
// with S_j the int8 dot of sub-block j.
//
// A K stage is half a super-block (4 sub-blocks, 128 elements). Per stage the
// workgroup stages into LDS:
//   * activation int8 rows as they are, copied by direct-to-LDS buffer loads
//     (no registers), and through registers the q8_K scale and (q4_K) the
//     eight 16-element bsums of the half as fp16 (|bsum| <= 2032 is exact in
//     fp16);
//   * weight values expanded to int8 (q4_K nibble 0..15 and the sub-block
//     scale digits; iq2_xxs two planes of the scaled value), and the fp16
//     scales.
// q4_K: sc (0..63) = 8*h + l with octal digits h, l. Two int8 weight planes
// q*l and q*h (both <= 105) are formed per fragment with one packed 16-bit
// multiply per dword (the byte products cannot carry), and two int8 MFMAs per
// sub-block accumulate S_L and S_H over the whole super-block, so IS = 8*S_H +
// S_L with no per-sub-block VALU work. IM is one fp16 MFMA per stage over the
// bsums and the mins (exact: every product and partial sum is an integer below
// 2^24).
// iq2_xxs: the staged value is the grid value times its sub-block scale,
// w' = sign * mag * (2 s + 1) with |w'| <= 43 * 31 = 1333, split as
// w' = 128 * hi + lo with lo in 0..127 and hi in -11..10 (both int8). Two
// int8 MFMAs per sub-block accumulate S_LO and S_HI over the whole
// super-block, so IS = 128 * S_HI + S_LO exactly, again with no per-sub-block
// VALU work. The split is a byte lookup (v_perm) into a per-scale table of the
// six (lo, hi) pairs of +-8, +-25, +-43 times the scale.
// A diagnostic instantiation writes the int32 super-block sums instead of C.
#include "device_common.h"
#include "kernels.h"
#include "pfng_iq2xxs_grid.h"

namespace pfng {

namespace {

__constant__ uint16_t kIq2GridCodes[256] = PFNG_IQ2XXS_GRID_CODES_INIT;

enum class Kq { Q4K, IQ2 };

// BM x BN workgroup tile, WM x WN waves over it, the 4 sub-blocks of each
// stage divided among WK waves, and WS slices of such waves that take every
// WS-th super-block each (each slice stages its own super-blocks in its own
// LDS buffers). WK * WS > 1: the partial accumulators are added through LDS
// at the end, in a fixed order.
template <Kq T, int BM, int BN, int WM, int WN, int WK = 1, int WS = 1>
struct KqConfig {
    static constexpr Kq kType = T;
    static constexpr bool kQ4K = T == Kq::Q4K;
    static constexpr int kBM = BM, kBN = BN, kWM = WM, kWN = WN, kWK = WK, kWS = WS;
    static constexpr int kThreads = 64 * WM * WN * WK;  // threads of one slice
    static constexpr int TM = BM / WM / 32;  // 32x32 tiles per wave along m
    static constexpr int TN = BN / WN / 32;  // along n
    static constexpr int kSub = 4;                    // sub-blocks per stage
    static constexpr int kWaveSub = kSub / WK;        // sub-blocks per stage of one wave
    static constexpr int kRowStride = kSub * 32 + 16;  // LDS bytes per int8 row (+ pad against bank conflicts)
    // A stage's activation rows of one slice, [BM][kRowStride] int8: nine
    // 16-byte chunks per row (eight of data, the pad), 64 chunks per copy
    // instruction, the region padded to whole instructions
    static constexpr int kRowChunks = kRowStride / 16;
    static constexpr int kActCopies = (BM * kRowChunks + 63) / 64;
    static constexpr int kAqBytes = kActCopies * 1024;
    static constexpr int kWaves = kThreads / 64;  // waves of one slice
    static constexpr int kActCopiesPerWave = (kActCopies + kWaves - 1) / kWaves;
    // LDS layout of the rest of one stage buffer
    static constexpr int kAd = 0;                                   // fp32 [BM] activation scale
    static constexpr int kAb = kAd + BM * 4;                        // q4_K: fp16 [BM][8] bsums of the half
    static constexpr int kWq = kAb + (kQ4K ? BM * 16 : 0);          // int8 [BN][kRowStride] (iq2: the lo plane)
    static constexpr int kWq2 = kWq + BN * kRowStride;              // iq2: int8 [BN][kRowStride] hi plane
    static constexpr int kWs = kWq2 + (kQ4K ? 0 : BN * kRowStride); // q4_K: u32 [BN][4][2] digit pairs
    static constexpr int kWd = kWs + (kQ4K ? BN * 32 : 0);          // fp32 [BN] d (iq2: 0.125 * d)
    static constexpr int kWdm = kWd + BN * 4;                       // q4_K: fp32 [BN] dmin
    static constexpr int kWmin = kWdm + (kQ4K ? BN * 4 : 0);        // q4_K: fp16 [BN][8] mins, each twice
    static constexpr int kBufBytes = kWmin + (kQ4K ? BN * 16 : 0);
    // iq2 tables: 256 x 8 grid code bytes (0, 1, 2 for 8, 25, 43), 128 x 8
    // sign selector bytes (4 where the value is negative), and per scale s the
    // (lo, hi) byte pairs of the six signed products
    static constexpr int kSigns = 256 * 8;
    static constexpr int kScaleTab = kSigns + 128 * 8;
    static constexpr int kTabBytes = kQ4K ? 16 : kScaleTab + 16 * 16;
    // the partial accumulators' reduction reuses the even stages' activation array
    static constexpr int kRedBytes = (WK * WS - 1) * WM * WN * TM * TN * 16 * 64 * 4;
    static constexpr int kAct0Bytes = WS * kAqBytes > kRedBytes ? WS * kAqBytes : kRedBytes;
    static constexpr int kLdsBytes = kAct0Bytes + WS * kAqBytes + 2 * WS * kBufBytes + kTabBytes;
    static constexpr int kAllThreads = kThreads * WS;
    // global -> register tasks per stage: each activation row in kActE parts
    // (2 or 4) of its 128 int8 and 8 bsums, each weight row per sub-block
    static constexpr int kActE = BM * 2 >= kThreads ? 2 : kThreads / BM;
    static constexpr int kQsDw = 32 / kActE;  // activation dwords per task
    static constexpr int kBsDw = 4 / kActE;   // bsum dwords per task
    static constexpr int kActPT = BM * kActE / kThreads;
    static constexpr int kWPT = BN * kSub / kThreads;
    static_assert(TM >= 1 && TN >= 1, "tile too small");
    static_assert(kActE == 2 || kActE == 4, "activation rows split in 2 or 4 parts");
    static_assert(kActPT * kThreads == BM * kActE && kWPT * kThreads == BN * kSub, "tasks must split evenly");
    static_assert(kActPT >= 1 && kWPT >= 1, "every thread takes at least one task of each operand");
    static_assert(kAd % 16 == 0 && kAb % 16 == 0 && kWq % 16 == 0 && kWq2 % 16 == 0 && kWs % 16 == 0 && kWd % 16 == 0 &&
                      kWdm % 16 == 0 && kWmin % 16 == 0 && kBufBytes % 16 == 0,
                  "LDS regions 16-byte aligned");
    static_assert(kRowStride % 16 == 0 && kRowChunks % 2 == 1, "rows of an odd number of whole chunks");
    static_assert(kWaveSub * WK == kSub, "the stage's sub-blocks split evenly over the K-waves");
    static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one CU");
};

template <class C>
struct KqRegs {
    uint32_t ab[C::kActPT][C::kBsDw];  // 8 / kActE bsums (q4_K)
    float ad[C::kActPT];
    // q4_K: 16 nibble bytes + the 16-byte header (d, dmin, scales)
    // iq2_xxs: the two dwords covering the sub-block's 8 bytes as loaded, d,
    // the trailing half-word and whether the bytes start 2 past a dword (the
    // realignment waits for the store, so the loads are not waited on early)
    uint32_t wq[C::kWPT][C::kQ4K ? 4 : 2];
    uint32_t wh[C::kWPT][C::kQ4K ? 4 : 3];
};

constexpr int kQ8KBytes = 292, kQ4KBytes = 144, kIq2Bytes = 66;

// Byte offsets of a thread's load tasks from the tile's first row at the
// stage's super-block: fixed over the K loop (rows past the matrix edge are
// clamped to its last row), so each stage's loads are a uniform base plus
// these 32-bit offsets. BM * nb * 292 < 2^32 for every k up to kMaxTiledK
// (mfma_supported declines longer rows).
template <class C>
struct KqOffsets {
    uint32_t a[C::kActPT];  // activation row + part e's qs dwords (its scale and bsums are read)
    uint32_t w[C::kWPT];    // weight row + sub-block e (iq2_xxs: its first byte past d)
};

template <class C>
__device__ __forceinline__ KqOffsets<C> kq_offsets(int m, int n, int nb, int m0, int n0, int tid) {
    KqOffsets<C> o;
#pragma unroll
    for (int it = 0; it < C::kActPT; ++it) {
        const int task = tid + it * C::kThreads;
        const int row = m0 + task / C::kActE, e = task % C::kActE;
        const int lrow = row < m ? row : m - 1;
        o.a[it] = (uint32_t)(lrow - m0) * (uint32_t)nb * (uint32_t)kQ8KBytes + 4u * C::kQsDw * (uint32_t)e;
    }
#pragma unroll
    for (int it = 0; it < C::kWPT; ++it) {
        const int task = tid + it * C::kThreads;
        const int row = n0 + task / C::kSub, e = task % C::kSub;
        const int lrow = row < n ? row : n - 1;
        o.w[it] = (uint32_t)(lrow - n0) * (uint32_t)nb * (uint32_t)(C::kQ4K ? kQ4KBytes : kIq2Bytes) +
                  (uint32_t)(C::kQ4K ? 16 * e : 2 + 8 * e);
    }
    return o;
}

// Loads of stage (b, H): super-block b, half H. a_t / w_t: the tile's first
// activation / weight row (uniform). Rows are clamped at the matrix edge so
// that every load is unconditional and in bounds.
template <class C, int H>
__device__ __forceinline__ void kq_load(const uint8_t *__restrict__ a_t, const uint8_t *__restrict__ w_t, int b,
                                        const KqOffsets<C> &o, int tid, KqRegs<C> &r) {
    const uint8_t *a_st = a_t + (size_t)b * kQ8KBytes;
    const uint8_t *w_st = w_t + (size_t)b * (C::kQ4K ? kQ4KBytes : kIq2Bytes);
#pragma unroll
    for (int it = 0; it < C::kActPT; ++it) {
        const int task = tid + it * C::kThreads;
        const int e = task % C::kActE;
        const uint8_t *blk = a_st + o.a[it] - 4 * C::kQsDw * e;
        const uint32_t *bs = reinterpret_cast<const uint32_t *>(blk + 260 + 16 * H + 4 * C::kBsDw * e);
        if constexpr (C::kQ4K) {
#pragma unroll
            for (int i = 0; i < C::kBsDw; ++i) r.ab[it][i] = bs[i];
        }
        r.ad[it] = *reinterpret_cast<const float *>(blk);
    }
#pragma unroll
    for (int it = 0; it < C::kWPT; ++it) {
        const int task = tid + it * C::kThreads;
        const int e = task % C::kSub;
        if constexpr (C::kQ4K) {
            const uint8_t *sub16 = w_st + o.w[it];  // = block + 16 e
            const uint32_t *qs = reinterpret_cast<const uint32_t *>(sub16 + 16 + 64 * H);
            const uint32_t *hd = reinterpret_cast<const uint32_t *>(sub16 - 16 * e);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                r.wq[it][i] = qs[i];
                r.wh[it][i] = hd[i];
            }
        } else {
            // 66-byte blocks are only 2-byte aligned: read the covering dwords
            // and a trailing half-word, never past the sub-block's last byte
            const uint8_t *sb = w_st + o.w[it] + 32 * H;  // sub-block e of half H
            const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(sb) & 3);  // 0 or 2
            const uint32_t *p4 = reinterpret_cast<const uint32_t *>(sb - sh);
            r.wq[it][0] = p4[0];
            r.wq[it][1] = p4[1];
            r.wh[it][0] = *reinterpret_cast<const uint16_t *>(sb - 32 * H - 2 - 8 * e);
            r.wh[it][1] = *reinterpret_cast<const uint16_t *>(sb + 6);
            r.wh[it][2] = sh;
        }
    }
}

// One 16-byte direct-to-LDS buffer load per lane (64 lanes: 1 KB at dst). A
// plain function: inside a kernel template the 16-byte form of the builtin
// makes the host pass drop the kernel's launch stub.
__device__ __forceinline__ void kq_copy16(__amdgpu_buffer_rsrc_t r, uint8_t *dst, uint32_t voffset, uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)dst, 16, voffset, soffset, 0,
                                             0);
}

// One slice's direct-to-LDS copies of a stage's activation rows (half H of
// super-block b) into act + aoff: copy j's lane l moves chunk c = 64 j + l, row
// c / 9, column c % 9 (the pad column repeats column 7; lanes past the rows
// repeat the last chunk into the region's padding; rows past rows_valid
// repeat the last valid row). The copies are dealt round-robin over the
// slice's waves, every wave issuing the same number (a wave past the last
// copy repeats it: c3 28.9 against 29.3 us when such waves skip it).
template <class C, int H>
__device__ __forceinline__ void kq_act_copy(uint8_t *act, int aoff, __amdgpu_buffer_rsrc_t ra, int b, int wave,
                                            int lane, int rows_valid, int nb) {
#pragma unroll
    for (int i = 0; i < C::kActCopiesPerWave; ++i) {
        int j = wave + i * C::kWaves;
        if (j > C::kActCopies - 1) j = C::kActCopies - 1;  // repeats the last copy
        int ch = 64 * j + lane;
        if (ch > C::kBM * C::kRowChunks - 1) ch = C::kBM * C::kRowChunks - 1;
        const int row = ch / C::kRowChunks;
        int col = ch - row * C::kRowChunks;
        if (col > C::kRowChunks - 2) col = C::kRowChunks - 2;
        const int rr = row < rows_valid ? row : rows_valid - 1;
        const uint32_t off = (uint32_t)rr * (uint32_t)nb * (uint32_t)kQ8KBytes + 4u + 16u * (uint32_t)col;
        kq_copy16(ra, act + (aoff + j * 1024), off, (uint32_t)b * kQ8KBytes + 128u * H);
    }
}

// An LDS address as the array plus one opaque offset (plus constants). The
// compiler attaches an array's alias scope only to accesses a few address
// steps from the array, and makes an LDS access without it wait for every
// direct-to-LDS copy in flight; left alone, it splits offsets into chains of
// address steps.
template <class T, class B>
__device__ __forceinline__ T *lds_at(B *arr, int off) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm("" : "+v"(off));
#endif
    return reinterpret_cast<T *>(arr + off);
}

// Registers of a stage into the stage buffer at rest + roff.
template <class C>
__device__ __forceinline__ void kq_store(uint8_t *rest, int roff, const uint8_t *tab, int h, int tid,
                                         const KqRegs<C> &r) {
    const uint8_t *grid = tab;
    const uint8_t *signs = tab + C::kSigns;
    const uint8_t *scale_tab = tab + C::kScaleTab;
#pragma unroll
    for (int it = 0; it < C::kActPT; ++it) {
        const int task = tid + it * C::kThreads;
        const int row = task / C::kActE, e = task % C::kActE;
        *lds_at<float>(rest, roff + C::kAd + row * 4) = r.ad[it];  // every part writes the same value
        if constexpr (C::kQ4K) {
            uint32_t hb[C::kBsDw];
#pragma unroll
            for (int i = 0; i < C::kBsDw; ++i) {
                const _Float16 lo = (_Float16)(float)(int16_t)(r.ab[it][i] & 0xffffu);
                const _Float16 hi = (_Float16)(float)(int16_t)(r.ab[it][i] >> 16);
                hb[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
            }
            uint32_t *bdst = lds_at<uint32_t>(rest, roff + C::kAb + row * 16 + 4 * C::kBsDw * e);
#pragma unroll
            for (int i = 0; i < C::kBsDw; ++i) bdst[i] = hb[i];
        }
    }
#pragma unroll
    for (int it = 0; it < C::kWPT; ++it) {
        const int task = tid + it * C::kThreads;
        const int row = task / C::kSub, e = task % C::kSub;
        const int wrow = roff + C::kWq + row * C::kRowStride;  // the row's lo (iq2) or value plane
        if constexpr (C::kQ4K) {
            // bytes 16e..16e+15 of the half's 64 nibble bytes: pair p = e/2
            // holds local sub-block 2p (low nibbles) and 2p+1 (high nibbles),
            // elements 16*(e%2) .. +15
            const int p = e / 2, i0 = 16 * (e % 2);
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[i] = r.wq[it][i] & 0x0f0f0f0fu;
                hi[i] = (r.wq[it][i] >> 4) & 0x0f0f0f0fu;
            }
            uint4 *dst = lds_at<uint4>(rest, wrow + (2 * p) * 32 + i0);
            dst[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            dst[2] = make_uint4(hi[0], hi[1], hi[2], hi[3]);  // 32 bytes on: sub-block 2p + 1
            // scale digits and min of local sub-block e
            uint32_t sc, mn;
            q4_K_scale_min(r.wh[it], 4 * h + e, sc, mn);
            const uint32_t l = sc & 7u, hh = sc >> 3;
            *lds_at<uint2>(rest, roff + C::kWs + row * 32 + 8 * e) = make_uint2(l * 0x10001u, hh * 0x10001u);
            const uint32_t mh = __builtin_bit_cast(uint16_t, (_Float16)(float)mn);
            *lds_at<uint32_t>(rest, roff + C::kWmin + row * 16 + 4 * e) = mh | (mh << 16);
            float *dd = lds_at<float>(rest, roff + C::kWd + row * 4);
            dd[0] = fp16_to_f32(r.wh[it][0] & 0xffffu);
            dd[(C::kWdm - C::kWd) / 4] = fp16_to_f32(r.wh[it][0] >> 16);
        } else {
            // iq2_xxs sub-block (kernels/common/iq2_xxs.h:29-41): four groups of
            // 8 values. A value's selector byte is its grid code (0, 1, 2 for
            // magnitude 8, 25, 43) plus 4 where it is negative (bit j of
            // idx | parity(idx) << 7, idx the 7-bit field g of the last dword);
            // it picks the lo and hi bytes of w' = +-mag * (2 * (bits 28..31) + 1)
            // from the scale's table (x: lo of the positive products, y: lo of
            // the negative ones, z / w: the hi bytes)
            const uint32_t d0 = r.wq[it][0], d1 = r.wq[it][1];
            const bool sh = r.wh[it][2] != 0;
            const uint32_t gidx = sh ? __builtin_amdgcn_alignbyte(d1, d0, 2) : d0;
            const uint32_t ss = sh ? ((d1 >> 16) | (r.wh[it][1] << 16)) : d1;
            const uint4 tab = *reinterpret_cast<const uint4 *>(scale_tab + 16 * (ss >> 28));
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint2 code = *reinterpret_cast<const uint2 *>(grid + ((gidx >> (8 * g)) & 0xffu) * 8);
                const uint2 neg = *reinterpret_cast<const uint2 *>(signs + ((ss >> (7 * g)) & 0x7fu) * 8);
                const uint32_t s0 = code.x | neg.x, s1 = code.y | neg.y;
                lo[2 * g] = __builtin_amdgcn_perm(tab.y, tab.x, s0);
                lo[2 * g + 1] = __builtin_amdgcn_perm(tab.y, tab.x, s1);
                hi[2 * g] = __builtin_amdgcn_perm(tab.w, tab.z, s0);
                hi[2 * g + 1] = __builtin_amdgcn_perm(tab.w, tab.z, s1);
            }
            uint4 *dlo = lds_at<uint4>(rest, wrow + 32 * e), *dhi = dlo + (C::kWq2 - C::kWq) / 16;
            dlo[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            dlo[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
            dhi[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            dhi[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            *lds_at<float>(rest, roff + C::kWd + row * 4) = 0.125f * fp16_to_f32(r.wh[it][0]);
        }
    }
}

// Per-wave accumulators.
template <class C>
struct KqAcc {
    f32x16 acc[C::TM][C::TN];  // fp32 output
    i32x16 s0[C::TM][C::TN];   // q4_K: S_L; iq2_xxs: S_LO
    i32x16 s1[C::TM][C::TN];   // q4_K: S_H; iq2_xxs: S_HI
    f32x16 im[C::TM][C::TN];   // q4_K: IM (exact integers)
};

// Sub-block sums of one stage (half H of the super-block) for one wave: its
// kWaveSub sub-blocks tb .. tb + kWaveSub - 1 (tb a multiple of kWaveSub).
// The stage's activation rows at act + aoff, the rest of its buffer at
// rest + roff (every LDS address the array plus one offset, as in kq_store).
template <class C, int H>
__device__ __forceinline__ void kq_compute(const uint8_t *act, int aoff, const uint8_t *rest, int roff, KqAcc<C> &A,
                                           int tb, int lane, int wave_m, int wave_n) {
    const int li = lane & 31, lh = lane >> 5;
    const uint8_t *aq = lds_at<const uint8_t>(act, aoff + (wave_m * C::TM * 32 + li) * C::kRowStride + lh * 16);
    const uint8_t *wq =
        lds_at<const uint8_t>(rest, roff + C::kWq + (wave_n * C::TN * 32 + li) * C::kRowStride + lh * 16);
    const int wrow = wave_n * C::TN * 32 + li;
    if constexpr (C::kQ4K) {
#pragma unroll
        for (int j = 0; j < C::kWaveSub; ++j) {
            const int t = tb + j;
            i32x4 av[C::TM], vl[C::TN], vh[C::TN];
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
                av[tm] = *reinterpret_cast<const i32x4 *>(aq + tm * 32 * C::kRowStride + t * 32);
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const i32x4 v = *reinterpret_cast<const i32x4 *>(wq + tn * 32 * C::kRowStride + t * 32);
                // digit pair (l, h) of sub-block t, each replicated in both 16-bit halves
                const uint2 d = lds_at<const uint2>(rest, roff + C::kWs + wrow * 32)[(tn * 32 * 32 + 8 * t) / 8];
                vl[tn] = mul_planes(v, d.x);
                vh[tn] = mul_planes(v, d.y);
            }
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < C::TN; ++tn) {
                    const bool first = H == 0 && j == 0;
                    A.s0[tm][tn] = mfma_i8_32x32x32(av[tm], vl[tn], first ? (i32x16){} : A.s0[tm][tn]);
                    A.s1[tm][tn] = mfma_i8_32x32x32(av[tm], vh[tn], first ? (i32x16){} : A.s1[tm][tn]);
                }
        }
        // IM over the half's 8 bsums: lane supplies row li and k = 4*lh .. 4*lh+3,
        // i.e. the bsums of sub-blocks 2*lh and 2*lh+1; lanes whose sub-blocks
        // belong to another K-wave contribute zero
        const bool mine = C::kWaveSub >= 4 || (2 * lh >= tb && 2 * lh < tb + C::kWaveSub);
        f16x4 ab[C::TM], wm[C::TN];
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
            ab[tm] =
                lds_at<const f16x4>(rest, roff + C::kAb + (wave_m * C::TM * 32 + li) * 16 + lh * 8)[tm * 32 * 2];
#pragma unroll
        for (int tn = 0; tn < C::TN; ++tn) {
            wm[tn] = lds_at<const f16x4>(rest, roff + C::kWmin + wrow * 16 + lh * 8)[tn * 32 * 2];
            if (!mine) wm[tn] = (f16x4){};
        }
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn)
                A.im[tm][tn] = mfma_f16_32x32x8(ab[tm], wm[tn], H == 0 ? (f32x16){} : A.im[tm][tn]);
    } else {
        // S_LO and S_HI over the lo and hi planes of the scaled values
        const uint8_t *wq2 = wq + (C::kWq2 - C::kWq);
#pragma unroll
        for (int j = 0; j < C::kWaveSub; ++j) {
            const int t = tb + j;
            i32x4 av[C::TM], wl[C::TN], wh[C::TN];
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
                av[tm] = *reinterpret_cast<const i32x4 *>(aq + tm * 32 * C::kRowStride + t * 32);
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                wl[tn] = *reinterpret_cast<const i32x4 *>(wq + tn * 32 * C::kRowStride + t * 32);
                wh[tn] = *reinterpret_cast<const i32x4 *>(wq2 + tn * 32 * C::kRowStride + t * 32);
            }
#pragma unroll
            for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < C::TN; ++tn) {
                    const bool first = H == 0 && j == 0;
                    A.s0[tm][tn] = mfma_i8_32x32x32(av[tm], wl[tn], first ? (i32x16){} : A.s0[tm][tn]);
                    A.s1[tm][tn] = mfma_i8_32x32x32(av[tm], wh[tn], first ? (i32x16){} : A.s1[tm][tn]);
                }
        }
    }
}

// End of super-block b: fold the exact sums into C (or write them out).
template <class C, bool kIsums>
__device__ __forceinline__ void kq_epilogue(const uint8_t *rest, int roff, KqAcc<C> &A, int32_t *isums, int m, int n,
                                            int nb, int m0, int n0, int b, int lane, int wave_m, int wave_n) {
    const int li = lane & 31, lh = lane >> 5;
    if constexpr (kIsums) {
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const int col = n0 + wave_n * C::TN * 32 + tn * 32 + li;
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int row = m0 + wave_m * C::TM * 32 + tm * 32 + mfma_row(lane, q);
                    if (row < m && col < n) {
                        const size_t o = ((size_t)row * n + col) * nb + b;
                        if constexpr (C::kQ4K) {
                            isums[2 * o] = 8 * A.s1[tm][tn][q] + A.s0[tm][tn][q];
                            isums[2 * o + 1] = (int32_t)A.im[tm][tn][q];
                        } else {
                            isums[o] = 128 * A.s1[tm][tn][q] + A.s0[tm][tn][q];
                        }
                    }
                }
            }
    } else {
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm) {
            // activation scales of the lane's 16 rows: rows 8g + 4lh + 0..3
            f32x4 ad4[4];
            if constexpr (C::kQ4K) {
                const f32x4 *adp =
                    lds_at<const f32x4>(rest, roff + C::kAd + 4 * (wave_m * C::TM * 32 + tm * 32 + 4 * lh));
#pragma unroll
                for (int g = 0; g < 4; ++g) ad4[g] = adp[2 * g];
            }
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const int wr = wave_n * C::TN * 32 + tn * 32 + li;
                const float *dp = lds_at<const float>(rest, roff + C::kWd + 4 * wr);
                const float d = dp[0];
                if constexpr (C::kQ4K) {
                    const float dmin = dp[(C::kWdm - C::kWd) / 4];
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const int is = 8 * A.s1[tm][tn][q] + A.s0[tm][tn][q];
                        const float x = fmaf(-dmin, A.im[tm][tn][q], d * (float)is);
                        A.acc[tm][tn][q] = fmaf(ad4[q / 4][q % 4], x, A.acc[tm][tn][q]);
                    }
                } else {
                    // P = ad (x) d on the matrix core: lane l supplies ad of row
                    // l % 32 and d of column l % 32 at K index l / 32, and the
                    // upper lanes' d is zero, so P[r][c] = ad_r * d_c, the
                    // correctly rounded product
                    const float adl =
                        *lds_at<const float>(rest, roff + C::kAd + 4 * (wave_m * C::TM * 32 + tm * 32 + li));
                    const f32x16 pr = __builtin_amdgcn_mfma_f32_32x32x2f32(adl, lh ? 0.0f : d, (f32x16){}, 0, 0, 0);
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        A.acc[tm][tn][q] = fmaf(pr[q], (float)(128 * A.s1[tm][tn][q] + A.s0[tm][tn][q]), A.acc[tm][tn][q]);
                }
            }
        }
    }
}

template <class C, bool kIsums>
__global__ __launch_bounds__(C::kAllThreads, 2) void gemm_kq_kernel(const uint8_t *__restrict__ w,
                                                                    const uint8_t *__restrict__ a,
                                                                    float *__restrict__ c, int32_t *__restrict__ isums,
                                                                    int m, int n, int nb) {
    // The activation rows of the even and the odd stages are separate arrays,
    // as is the rest of the stage buffers: the compiler then waits, before
    // a stage's LDS reads, only for the copies into that stage's array, not
    // for those of the next stage, which are in flight meanwhile.
    __shared__ __align__(16) uint8_t act0[C::kAct0Bytes];
    __shared__ __align__(16) uint8_t act1[C::kWS * C::kAqBytes];
    __shared__ __align__(16) uint8_t rest0[C::kWS * C::kBufBytes];
    __shared__ __align__(16) uint8_t rest1[C::kWS * C::kBufBytes];
    __shared__ __align__(16) uint8_t tab[C::kTabBytes];
    const int lane = threadIdx.x & 63;
    // iq2_xxs grid codes (kernels/iq2_xxs-q8_K-RVV-common/ggml_min.h:69-134):
    // their address is fixed at load time, so their loads go out before
    // anything that needs a kernel argument, and the tables are built only
    // after the first stage's copies and loads have been issued: the codes'
    // trip from L2 overlaps the first stage's from HBM (iq2_xxs
    // 256x4096x4096 19.6 -> 19.4 us, c3 within noise)
    constexpr int kCodeIters = C::kQ4K ? 1 : (256 + C::kAllThreads - 1) / C::kAllThreads;
    uint32_t codes[kCodeIters];
    if constexpr (!C::kQ4K) {
#pragma unroll
        for (int i = 0; i < kCodeIters; ++i) {
            const int e = (int)threadIdx.x + i * C::kAllThreads;
            codes[i] = kIq2GridCodes[e < 256 ? e : 255];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // slice takes super-blocks slice, slice + WS, ...; slice and wave are
    // wave-uniform (the copies' LDS addresses go to a scalar register)
    const int slice = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / C::kThreads));
    const int tid = threadIdx.x % C::kThreads;  // thread index within the slice
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wk = wave / (C::kWM * C::kWN);   // which share of each stage's sub-blocks
    const int wmn = wave % (C::kWM * C::kWN);  // which TM x TN sub-tile
    const int wave_m = wmn / C::kWN;
    const int wave_n = wmn % C::kWN;
    const int tb = wk * C::kWaveSub;
    // n-fastest per XCD: right after the activation quantizer has rewritten
    // the q8_K rows, each XCD's L2 fetches only its own m-tiles' rows (c3
    // end to end 37.3 -> 35.8 us; the product alone within 1 %)
    const TileOrigin to = xcd_tile<1>(blockIdx.x, (m + C::kBM - 1) / C::kBM, (n + C::kBN - 1) / C::kBN);
    const int m0 = to.mi * C::kBM, n0 = to.ni * C::kBN;
    const int aoff = slice * C::kAqBytes, roff = slice * C::kBufBytes;  // the slice's part of each array
    // the iq2_xxs tables in LDS, from the codes loaded above
    auto build_tables = [&]() __attribute__((always_inline)) {
        // grid: per value one byte 0, 1 or 2 for the magnitude 8, 25 or 43
#pragma unroll
        for (int i = 0; i < kCodeIters; ++i) {
            const int e = (int)threadIdx.x + i * C::kAllThreads;
            if (e >= 256) break;
            const uint32_t code = codes[i];
            uint32_t v[2] = {0, 0};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j / 4] |= ((code >> (2 * j)) & 3u) << (8 * (j % 4));
            *reinterpret_cast<uint2 *>(tab + 8 * e) = make_uint2(v[0], v[1]);
        }
        // signs (the reference's ksigns_iq2xs, ggml_min.h:58-67: byte
        // idx | parity(idx) << 7): 4 in the byte of each negative value
        for (int e = threadIdx.x; e < 128; e += C::kAllThreads) {
            const uint32_t sgn = (uint32_t)e | ((__builtin_popcount((uint32_t)e) & 1u) << 7);
            uint32_t v[2] = {0, 0};
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j / 4] |= ((sgn >> j) & 1u) << (8 * (j % 4) + 2);
            *reinterpret_cast<uint2 *>(tab + C::kSigns + 8 * e) = make_uint2(v[0], v[1]);
        }
        // per 4-bit scale s: w' = +-mag * (2 s + 1) = 128 hi + lo, byte c of
        // the positive and byte c of the negative words for code c
        for (int e = threadIdx.x; e < 16; e += C::kAllThreads) {
            const int sc = 2 * e + 1;
            uint32_t lp = 0, ln = 0, hp = 0, hn = 0;
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const int p = (c == 0 ? 8 : (c == 1 ? 25 : 43)) * sc, q = -p;
                lp |= (uint32_t)(p & 127) << (8 * c);
                hp |= (uint32_t)((p >> 7) & 0xff) << (8 * c);
                ln |= (uint32_t)(q & 127) << (8 * c);
                hn |= (uint32_t)((q >> 7) & 0xff) << (8 * c);
            }
            *reinterpret_cast<uint4 *>(tab + C::kScaleTab + 16 * e) = make_uint4(lp, ln, hp, hn);
        }
    };

    KqAcc<C> A;
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j) A.acc[i][j] = (f32x16){};

    // Double-buffered LDS with one barrier per stage. Stage 2b+h is computed
    // from buffer h while the next stage's activation rows are copied into
    // the other buffer, its registers are stored there and the loads of the
    // stage after it are issued. Copies, stores and loads are unconditional
    // (the super-block index is clamped at the end); every slice runs the
    // same number of iterations, and one whose super-block is past the end
    // skips only the arithmetic. That check is only compiled into the one
    // iteration that can need it: a branch around the arithmetic in every
    // iteration made the compiler copy the just-loaded registers before the
    // barrier and so wait for the loads there. (Loads issued two stages
    // ahead, from a register set per half, measured no faster on c2/c3.)
    KqRegs<C> regs;
    const int last = nb - 1;
    const uint8_t *a_t = a + (size_t)m0 * nb * kQ8KBytes;
    const uint8_t *w_t = w + (size_t)n0 * nb * (C::kQ4K ? kQ4KBytes : kIq2Bytes);
    const KqOffsets<C> offs = kq_offsets<C>(m, n, nb, m0, n0, tid);
    const int rows_a = m - m0 < C::kBM ? m - m0 : C::kBM;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a_t, 0, (int)((uint32_t)rows_a * (uint32_t)nb * kQ8KBytes), 0x00020000);
    const int b0 = slice < nb ? slice : last;
    kq_act_copy<C, 0>(act0, aoff, ra, b0, wave, lane, rows_a, nb);
    kq_load<C, 0>(a_t, w_t, b0, offs, tid, regs);
    if constexpr (!C::kQ4K) {
        __builtin_amdgcn_sched_barrier(0);
        build_tables();
        __syncthreads();
    }
    kq_store<C>(rest0, roff, tab, 0, tid, regs);
    kq_load<C, 1>(a_t, w_t, b0, offs, tid, regs);
    __syncthreads();
    auto step = [&](int it, bool guard) __attribute__((always_inline)) {
        const int b = it * C::kWS + slice;
        const bool mine = !guard || b < nb;  // uniform across the slice's waves
        const int bn = b + C::kWS < nb ? b + C::kWS : last;
        __builtin_amdgcn_sched_barrier(0);
        kq_act_copy<C, 1>(act1, aoff, ra, b < nb ? b : last, wave, lane, rows_a, nb);
        __builtin_amdgcn_sched_barrier(0);
        if (mine) kq_compute<C, 0>(act0, aoff, rest0, roff, A, tb, lane, wave_m, wave_n);
        __builtin_amdgcn_sched_barrier(0);
        kq_store<C>(rest1, roff, tab, 1, tid, regs);
        __builtin_amdgcn_sched_barrier(0);
        kq_load<C, 0>(a_t, w_t, bn, offs, tid, regs);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        kq_act_copy<C, 0>(act0, aoff, ra, bn, wave, lane, rows_a, nb);
        __builtin_amdgcn_sched_barrier(0);
        if (mine) {
            kq_compute<C, 1>(act1, aoff, rest1, roff, A, tb, lane, wave_m, wave_n);
            kq_epilogue<C, kIsums>(rest1, roff, A, isums, m, n, nb, m0, n0, b, lane, wave_m, wave_n);
        }
        __builtin_amdgcn_sched_barrier(0);
        kq_store<C>(rest0, roff, tab, 0, tid, regs);
        __builtin_amdgcn_sched_barrier(0);
        kq_load<C, 1>(a_t, w_t, bn, offs, tid, regs);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    const int full = nb / C::kWS;  // iterations in which every slice has a super-block
    for (int it = 0; it < full; ++it) step(it, false);
    if (full * C::kWS < nb) step(full, true);

    if constexpr (!kIsums) {
        constexpr int kGroups = C::kWK * C::kWS;  // partial accumulators per output tile
        if constexpr (kGroups > 1) {
            // add the other groups' partials to group 0's (slice 0, wk 0), in
            // group order; the stage buffers are free after the last barrier
            constexpr int kRegs = C::TM * C::TN * 16;
            const int grp = slice * C::kWK + wk;
            float *red = reinterpret_cast<float *>(act0);
            if (grp > 0) {
                float *dst = red + ((grp - 1) * C::kWM * C::kWN + wmn) * kRegs * 64 + lane;
#pragma unroll
                for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
                        for (int r = 0; r < 16; ++r) dst[((tm * C::TN + tn) * 16 + r) * 64] = A.acc[tm][tn][r];
            }
            __syncthreads();
            if (grp > 0) return;
#pragma unroll
            for (int g2 = 1; g2 < kGroups; ++g2) {
                const float *src = red + ((g2 - 1) * C::kWM * C::kWN + wmn) * kRegs * 64 + lane;
#pragma unroll
                for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
                    for (int tn = 0; tn < C::TN; ++tn)
#pragma unroll
                        for (int r = 0; r < 16; ++r) A.acc[tm][tn][r] += src[((tm * C::TN + tn) * 16 + r) * 64];
            }
        }
        const int li = lane & 31;
#pragma unroll
        for (int tm = 0; tm < C::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < C::TN; ++tn) {
                const int col = n0 + wave_n * C::TN * 32 + tn * 32 + li;
                if (col < n) {
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const int row = m0 + wave_m * C::TM * 32 + tm * 32 + mfma_row(lane, q);
                        if (row < m) store_through(&c[(size_t)row * n + col], A.acc[tm][tn][q]);
                    }
                }
            }
    }
}

template <class C, bool kIsums>
hipError_t launch_kq(const void *w, const void *a, float *c, int32_t *isums, int64_t m, int64_t n, int64_t k,
                     hipStream_t stream) {
    const dim3 grid((unsigned)(((n + C::kBN - 1) / C::kBN) * ((m + C::kBM - 1) / C::kBM)));
    hipLaunchKernelGGL((gemm_kq_kernel<C, kIsums>), grid, dim3(C::kAllThreads), 0, stream,
                       static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(a), c, isums, (int)m, (int)n,
                       (int)(k / 256));
    return hipGetLastError();
}

// large problems: 128 x 64 tiles, 4 waves of 64 x 32
template <Kq T>
using KqBig = KqConfig<T, 128, 64, 2, 2>;
// small problems: 32 x 32 tiles. q4_K: 2 waves each taking 2 of the stage's 4
// sub-blocks (its accuracy bound is per element, so partial super-block sums
// may be scaled separately). iq2_xxs: one wave, since its bound is per
// super-block: the integer sum must be complete before it is scaled, or
// partial sums that nearly cancel would be rounded against a small total.
template <Kq T>
using KqTiny = KqConfig<T, 32, 32, 1, 1, T == Kq::Q4K ? 2 : 1>;
// decode batches: the Tiny tile with 4 or 2 slices of whole super-blocks, so
// that a few hundred output tiles still keep several waves on every CU (the
// slices split the K range at super-block boundaries, which the iq2_xxs bound
// allows)
template <Kq T>
using KqMid = KqConfig<T, 32, 32, 1, 1, T == Kq::Q4K ? 2 : 1, 4>;
template <Kq T>
using KqMid2 = KqConfig<T, 32, 32, 1, 1, T == Kq::Q4K ? 2 : 1, 2>;

// the 128 x 64 and 64 x 64 tiles with 2 slices: 8 waves per workgroup where
// the tiles alone give about one workgroup per CU
template <Kq T>
using KqBigS2 = KqConfig<T, 128, 64, 2, 2, 1, 2>;
template <Kq T>
using KqSmallS2 = KqConfig<T, 64, 64, 2, 2, 1, 2>;

enum { kCfgBig = 0, kCfgTiny = 2, kCfgMid = 3, kCfgMid2 = 4, kCfgBigS2 = 5, kCfgSmallS2 = 6, kCfgWhole = 7 };

int64_t tiles_of(int64_t m, int64_t n, int64_t bm, int64_t bn) { return ((m + bm - 1) / bm) * ((n + bn - 1) / bn); }

template <Kq T>
hipError_t dispatch(const void *w, const void *a, float *c, const MfmaPlan &plan, int64_t m, int64_t n, int64_t k,
                    hipStream_t stream) {
    switch (plan.config) {
    case kCfgBig: return launch_kq<KqBig<T>, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgMid: return launch_kq<KqMid<T>, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgMid2: return launch_kq<KqMid2<T>, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgBigS2: return launch_kq<KqBigS2<T>, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgSmallS2: return launch_kq<KqSmallS2<T>, false>(w, a, c, nullptr, m, n, k, stream);
    case kCfgWhole: return launch_q4_K_small(w, a, c, m, n, k, stream);
    default: return launch_kq<KqTiny<T>, false>(w, a, c, nullptr, m, n, k, stream);
    }
}

}  // namespace

// Tile choice (measured on MI355X, 256 CUs, n = 4096 and the baseline
// shapes): q4_K at k = 1024 or 1536 with half to one 32 x 96 tile per CU: the
// whole-K tiles of gemm_small.hip (c2: 7.60 against 8.59 us for the 64 x 64
// tiles with 2 slices); 128 x 64 tiles at two or more per CU; with 2
// super-block slices at one or more per CU (c3); 64 x 64 tiles with 2 slices
// from half a tile per CU (q4_K) or three quarters (iq2_xxs) (c2 before the
// whole-K tiles: 9.1 instead of 11.3 us); below that the 32 x 32 tile with the
// most slices (4, 2, 1) that keeps the waves at or under 8 per CU (more slices
// only added barrier and staging work). The block-sum diagnostic of the
// whole-K plan reports the 64 x 64 two-slice tiles' sums (the whole-K tiles
// split super-blocks between K slices and add the parts only in fp32).
MfmaPlan plan_kquant(int type, int64_t m, int64_t n, int64_t k, int cus) {
    MfmaPlan p;
    const int64_t c = cus;
    const bool q4k = type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K;
    const int64_t wk = q4k ? 2 : 1;  // KqTiny's K-waves
    const int64_t t32 = tiles_of(m, n, 32, 32), t64 = tiles_of(m, n, 64, 64), t128 = tiles_of(m, n, 128, 64);
    const int64_t t96 = tiles_of(m, n, 32, 96);
    if (q4k && q4_K_small_supported(k) && 2 * t96 >= c && t96 <= c)
        p.config = kCfgWhole;
    else if (t128 >= 2 * c)
        p.config = kCfgBig;
    else if (t128 >= c)
        p.config = kCfgBigS2;
    else if (4 * t64 >= (q4k ? 2 : 3) * c)
        p.config = kCfgSmallS2;
    else if (t32 * 4 * wk <= 8 * c)
        p.config = kCfgMid;
    else if (t32 * 2 * wk <= 8 * c)
        p.config = kCfgMid2;
    else
        p.config = kCfgTiny;
    return p;
}

hipError_t launch_kquant_mul_mat(int type, const void *w, const void *a, float *c, int64_t m, int64_t n, int64_t k,
                                 const MfmaPlan &plan, hipStream_t stream) {
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) return dispatch<Kq::Q4K>(w, a, c, plan, m, n, k, stream);
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) return dispatch<Kq::IQ2>(w, a, c, plan, m, n, k, stream);
    return hipErrorInvalidValue;
}

// The block-sum diagnostic of a configuration. K-waves (WK > 1, q4_K's
// 32 x 32 tiles) split each super-block's sub-blocks and only meet in the fp32
// reduction, so their integer sums are reported by the same tile and slices
// with one K-wave; every other configuration reports its own sums.
template <class C>
using KqIsums = KqConfig<C::kType, C::kBM, C::kBN, C::kWM, C::kWN, 1, C::kWS>;

template <Kq T>
hipError_t dispatch_isums(const void *w, const void *a, int32_t *out, const MfmaPlan &plan, int64_t m, int64_t n,
                          int64_t k, hipStream_t stream) {
    switch (plan.config) {
    case kCfgBig: return launch_kq<KqIsums<KqBig<T>>, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgBigS2: return launch_kq<KqIsums<KqBigS2<T>>, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgSmallS2:
    case kCfgWhole: return launch_kq<KqIsums<KqSmallS2<T>>, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgMid: return launch_kq<KqIsums<KqMid<T>>, true>(w, a, nullptr, out, m, n, k, stream);
    case kCfgMid2: return launch_kq<KqIsums<KqMid2<T>>, true>(w, a, nullptr, out, m, n, k, stream);
    default: return launch_kq<KqIsums<KqTiny<T>>, true>(w, a, nullptr, out, m, n, k, stream);
    }
}

hipError_t launch_kquant_block_isums(int type, const void *w, const void *a, int32_t *out, int64_t m, int64_t n,
                                     int64_t k, const MfmaPlan &plan, hipStream_t stream) {
    if (type == PFNG_WEIGHT_Q4_K_ACTIVATION_Q8_K) return dispatch_isums<Kq::Q4K>(w, a, out, plan, m, n, k, stream);
    if (type == PFNG_WEIGHT_IQ2_XXS_ACTIVATION_Q8_K) return dispatch_isums<Kq::IQ2>(w, a, out, plan, m, n, k, stream);
    return hipErrorInvalidValue;
}

}  // namespace pfng
