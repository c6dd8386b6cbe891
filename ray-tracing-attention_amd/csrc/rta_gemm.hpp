// rta_gemm.hpp -- batched (>= 8 rows) dequant-fused readout on the gfx950 matrix cores.
//
// y[b, r] = sum_k W[r, k] x[b, k] for up to 32 x rows per launch with
// v_mfma_f32_16x16x32_f16 (fp32 accumulation).
//
//   x (A operand), prepared by xprep_kernel per (batch row, superblock of 256
//   columns): a power-of-two scale s puts max|x s| in [2^13, 2^14); x s is split
//   into binary16 hi + lo (22 significant bits) and both are multiplied in.  The
//   group sums the formats need (sum x over 32 for the Q4_K minimum, over 16 for
//   the Q6_K -32 offset) are prepared the same way, already in A-operand order.
//
//   Weights (B operand) are built in registers as exact binary16 values with one
//   packed multiply per two codes: a code c in the low bits of a half is the
//   subnormal c * 2^-24, and
//     Q4_K  low nibble  (c 2^-24) * (sc 2^10) = c sc 2^-14   (c sc <= 945)
//           high nibble (16 c 2^-24) * (sc 2^6) = c sc 2^-14
//     Q6_K  (4 c 2^-24) * (sc 2^8) = c sc 2^-14  (exact for |c sc| <= 2048; beyond,
//           |sc| > 32, it rounds to 11 bits, <= 2^-12 relative; the -32 offset is
//           applied exactly through the group sums)
//   so every product handed to the matrix cores is a normal binary16 (or zero).
//   The masks deliver code pairs (k, k+2); x is stored in the same order inside
//   every 8-value segment (slots 0..7 hold k = 0,2,1,3,4,6,5,7), and a common
//   permutation of k leaves the contraction unchanged.
//   Per superblock the MFMAs accumulate across all groups; the superblock's
//   scale d, the minimum / offset terms (one more MFMA over the group sums) and
//   the 1/s of x are applied once per superblock.
//
//   Lane l of a wave owns weight row l%16 / k segment 8*(l/16) (B operand), batch
//   row l%16 / k segment (A operand), and outputs (batch 4*(l/16)+e, row l%16).
//
//   Work split: the K range is cut into slabs of up to 8 (16 x rows) or 4 (32 x
//   rows) superblocks.  A workgroup (8 waves, one per CU) loads its slab of x into
//   LDS once; after that its waves run independently over tiles of 16*RT weight
//   rows, each loading the next superblock's weights into registers while the
//   current one is multiplied.  With one slab the kernel applies the epilogue
//   itself; with more it writes per-slab partial sums that gemm_reduce_kernel adds
//   in slab order (deterministic).
//
// Equivalent reference: the batched projection pipelines (optical_resident.cpp:168,343,
// matrixRows 4/8/16) and resident_batch2.comp (which accumulates in fp16; not copied).
#pragma once
#include <type_traits>
#include "rta_gemv.hpp"

namespace rta {


constexpr int kMaxBatchTile = 32;  // batch rows per GEMM launch
constexpr int kXStride = 256 + 8;  // f16 per staged x row (8 of padding spread the LDS banks)
constexpr int kGemmWaves = 8;      // waves per workgroup
constexpr int kSlabRowSb = 128;    // LDS holds (x rows) * (superblocks) <= 128

struct GemmX {           // prepared x (workspace), batch padded to 32
    _Float16* hi;        // [32][cols]          x s, k-permuted inside 8-segments
    _Float16* lo;        // [32][cols]
    h8_t* g;             // [32][cols/256][4]   group-sum A operand per k segment
    float* inv;          // [32][cols/256]      1/s (0 for padding rows)
};

// ---------------------------------------------------------------- x prep ----
// Group-sum operand layouts (8 f16 per lane segment s = 0..3 of the superblock):
//   kXpQ4Row   s0 = hi of 32-groups 0..7, s1 = lo of 0..7, s2 = s3 = 0
//   kXpQ6Row   s0 = hi of 16-groups 0..7, s1 = hi of 8..15, s2 = lo of 0..7, s3 = lo of 8..15
//   kXpQ4Tile  s = [hi, lo of 32-group 2s, hi, lo of 2s+1, 0, 0, 0, 0]
//   kXpQ6Tile  s = [hi, lo of 16-group g(q)] for q = 0..3, g(q) = 8 (s/2) + 2 q + s%2
enum { kXpQ4Row = 0, kXpQ6Row = 1, kXpQ4Tile = 2, kXpQ6Tile = 3 };

// Block: 64 threads = 2 batch rows x 32 threads; thread = 8 consecutive columns of
// superblock blockIdx.x.
template <int LAYOUT>
__global__ void __launch_bounds__(64) xprep_kernel(const float* __restrict__ x, int cols, int batch, GemmX p) {
    const int lane = threadIdx.x, sb = blockIdx.x;
    const int b = blockIdx.y * 2 + (lane >> 5), t = lane & 31;
    const int nsb = cols >> 8;
    const int c0 = sb * 256 + 8 * t;
    float v[8];
    if (b < batch) {
        const float4* src = reinterpret_cast<const float4*>(x + (int64_t)b * cols + c0);
        const float4 a = src[0], c = src[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    m = group_max(m, 32);   // within 32 lanes
    const int e = operand_exponent(m);
    const float s = ldexpf(1.0f, 14 - e);        // m * s in [2^13, 2^14)
    if (t == 0) p.inv[(int64_t)b * nsb + sb] = b < batch ? ldexpf(1.0f, e - 14) : 0.0f;
    constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    _Float16 hi[8], lo[8];
    float sum8 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float w = v[perm[i]] * s;
        hi[i] = (_Float16)w;
        lo[i] = (_Float16)(w - (float)hi[i]);
        sum8 += v[i] * s;
    }
    const int64_t at = (int64_t)b * cols + c0;
    *reinterpret_cast<h8_t*>(p.hi + at) = h8_t{hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6], hi[7]};
    *reinterpret_cast<h8_t*>(p.lo + at) = h8_t{lo[0], lo[1], lo[2], lo[3], lo[4], lo[5], lo[6], lo[7]};
    _Float16* g = reinterpret_cast<_Float16*>(p.g + ((int64_t)b * nsb + sb) * 4);   // 32 f16
    const float s16 = sum8 + dpp_mov<0xB1>(sum8);
    const float s32 = s16 + dpp_mov<0x4E>(s16);
    if constexpr (LAYOUT == kXpQ6Row || LAYOUT == kXpQ6Tile) {
        if ((t & 1) == 0) {   // 16-group u = t / 2
            const int u = t >> 1;
            const float w = s16 * (1.0f / 16.0f);
            const _Float16 h = (_Float16)w, l = (_Float16)(w - (float)h);
            if constexpr (LAYOUT == kXpQ6Row) {
                g[8 * (u >> 3) + (u & 7)] = h;
                g[16 + 8 * (u >> 3) + (u & 7)] = l;
            } else {   // u = 8 hh + 2 q + sg -> segment 2 hh + sg, slot 2 q
                const int seg = 2 * (u >> 3) + (u & 1), q = (u >> 1) & 3;
                g[8 * seg + 2 * q] = h;
                g[8 * seg + 2 * q + 1] = l;
            }
        }
    } else {
        const int q = t >> 2;  // 32-group
        if ((t & 3) == 0) {
            const float w = s32 * (1.0f / 32.0f);
            const _Float16 h = (_Float16)w, l = (_Float16)(w - (float)h);
            if constexpr (LAYOUT == kXpQ4Row) {
                g[q] = h;
                g[8 + q] = l;
            } else {
                g[8 * (q >> 1) + 2 * (q & 1)] = h;
                g[8 * (q >> 1) + 2 * (q & 1) + 1] = l;
            }
        } else if ((t & 3) == 1) {   // the zero slots
            if constexpr (LAYOUT == kXpQ4Row) {
                g[16 + q] = (_Float16)0.0f;
                g[24 + q] = (_Float16)0.0f;
            } else {
                g[8 * (q >> 1) + 4 + 2 * (q & 1)] = (_Float16)0.0f;
                g[8 * (q >> 1) + 5 + 2 * (q & 1)] = (_Float16)0.0f;
            }
        }
    }
}


// -------------------------------------------------------- weight operand ----
// Per lane: row l%16 of one 16-row tile, k segment s = l/16 of every 32-value chunk.
struct Q4KMma {
    static constexpr int kBlock = 144;
    struct Raw { uint4 hdr; uint2 q[4]; };   // q[j] = bytes 16+32j+8s .. +8
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ blk, int s, Raw& r) {
        r.hdr = *reinterpret_cast<const uint4*>(blk);
#pragma unroll
        for (int j = 0; j < 4; ++j) r.q[j] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * j + 8 * s);
    }
};

struct Q6KMma {
    static constexpr int kBlock = 210;
    // half h: ql runs at 64h + 8s and 64h + 32 + 8s, qh run at 128 + 32h + 8s (8 bytes
    // each), loaded as 3 dwords from the 4-byte aligned address at or below; scales; d.
    // Every dword read overlaps the 210-byte block (blocks are 2-byte aligned).
    struct Raw { uint32_t a[2][3], b[2][3], h[2][3]; uint32_t sc[5]; uint32_t d; uint32_t mis; };
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ blk, int s, Raw& r) {
        // aligned down by pointer arithmetic, which keeps the global address space
        const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const uint32_t* a = reinterpret_cast<const uint32_t*>(blk - mis);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int ia = (64 * hh + 8 * s) >> 2, ib = (64 * hh + 32 + 8 * s) >> 2, ih = (128 + 32 * hh + 8 * s) >> 2;
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                r.a[hh][i] = a[ia + i];
                r.b[hh][i] = a[ib + i];
                r.h[hh][i] = a[ih + i];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) r.sc[i] = a[48 + i];          // bytes 192..207 (+mis)
        r.sc[4] = a[48 + 3 + (mis ? 1 : 0)];                     // bytes 208..211 only if 2-aligned
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
        r.mis = mis;
    }
};

// Static LDS of the GEMM: the x slab (hi and lo planes), group-sum operands, 1/s.
template <int NBT>
struct GemmSmem {
    static constexpr int kRows = 16 * NBT;
    static constexpr int kSb = kSlabRowSb / kRows;   // superblocks per slab
    _Float16 x[kSb][2][kRows][kXStride];
    h8_t g[kSb][kRows][4];
    float inv[kSb][kRows];
};

template <int FMT, int RT, int NBT, int MODE>
__global__ void __launch_bounds__(64 * kGemmWaves) gemm_mfma_kernel(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, const int64_t row_bytes, const int rows,
    const int cols, const GemmX xp, const int batch, float* __restrict__ y, float* __restrict__ part,
    float* __restrict__ pmax, const int sb_per_slab, const int wgs_per_slab) {
    constexpr bool kQ4 = FMT == RTA_Q4_K;
    using Fmt = typename std::conditional<kQ4, Q4KMma, Q6KMma>::type;
    using Raw = typename Fmt::Raw;
    using Smem = GemmSmem<NBT>;
    constexpr int kRows = Smem::kRows;
    constexpr int kTile = 16 * RT;
    __shared__ Smem sm;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: scalar loop control
    const int slab = blockIdx.x / wgs_per_slab, pos = blockIdx.x - slab * wgs_per_slab;
    const int nslab = gridDim.x / wgs_per_slab;
    const int nsbt = cols >> 8;
    const int sb0 = slab * sb_per_slab;
    const int nsb = min(sb_per_slab, nsbt - sb0);
    const int s = lane >> 4, li = lane & 15;
    const int total_rows = MODE == kSwiglu ? 2 * rows : rows;

    // ---- this wave's tiles: tg = gw, gw + nw, ...; iteration = (tile, superblock)
    const int gw = pos * kGemmWaves + wave, nw = wgs_per_slab * kGemmWaves;
    const int ntg = (total_rows + kTile - 1) / kTile;
    const int my_tiles = gw < ntg ? (ntg - 1 - gw) / nw + 1 : 0;
    const int nit = my_tiles * nsb;

    auto load_w = [&](int it, Raw* dst) {
        const int tgi = it / nsb, sbl = it - tgi * nsb;
        const int tg = gw + tgi * nw;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            // In kSwiglu virtual row v is gate row v/2 (v even) or up row v/2 (v odd).
            // Rows past the end are clamped, computed and dropped.
            const int v = min(tg * kTile + t * 16 + li, total_rows - 1);
            const uint8_t* rowp;
            if constexpr (MODE == kSwiglu) rowp = ((v & 1) ? w2 : w) + (int64_t)(v >> 1) * row_bytes;
            else rowp = w + (int64_t)v * row_bytes;
            Fmt::load(rowp + (int64_t)(sb0 + sbl) * Fmt::kBlock, s, dst[t]);
        }
    };

    // Weights are prefetched DEPTH - 1 superblocks ahead through rotating register
    // buffers; the first loads are issued before the x slab is staged.
    // Loads are unconditional (indices clamped to the last iteration) so that the
    // outstanding-load counts the compiler waits on are static.
    constexpr int DEPTH = kQ4 ? 3 : 2;
    Raw buf[DEPTH][RT];
    if (nit > 0) {
#pragma unroll
        for (int d = 0; d < DEPTH - 1; ++d) load_w(min(d, nit - 1), buf[d]);
    }

    // ---- x slab -> LDS (the only barrier of the kernel).  Every load of a thread is
    // issued before the first LDS store, so the slab costs one memory round trip.
    {
        constexpr int kThreads = 64 * kGemmWaves;
        constexpr int kPer = Smem::kSb * 2 * kRows * 32 / kThreads;   // 16-byte chunks per thread
        const int nchunk = nsb * 2 * kRows * 32;
        uint4 tmp[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {   // unconditional (clamped) loads
            const int i = min(tid + k * kThreads, nchunk - 1);
            const int c8 = i & 31, r = (i >> 5) % kRows, plane = ((i >> 5) / kRows) & 1, sbl = i / (64 * kRows);
            tmp[k] = *reinterpret_cast<const uint4*>((plane ? xp.lo : xp.hi) + (int64_t)r * cols +
                                                     (int64_t)(sb0 + sbl) * 256 + 8 * c8);
        }
        static_assert(Smem::kSb * kRows * 4 <= kThreads && Smem::kSb * kRows <= kThreads, "one operand per thread");
        const int gi = min(tid, nsb * kRows * 4 - 1), ii = min(tid, nsb * kRows - 1);
        const int gq = gi & 3, gr = (gi >> 2) % kRows, gs = gi / (4 * kRows);
        const h8_t gv = xp.g[((int64_t)gr * nsbt + sb0 + gs) * 4 + gq];
        const int ir = ii % kRows, is = ii / kRows;
        const float iv = xp.inv[(int64_t)ir * nsbt + sb0 + is];
        // Stores are unconditional too (threads past the end rewrite the last chunk with
        // the same data), so that the compiler cannot sink the loads next to them.
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int i = min(tid + k * kThreads, nchunk - 1);
            const int c8 = i & 31, r = (i >> 5) % kRows, plane = ((i >> 5) / kRows) & 1, sbl = i / (64 * kRows);
            *reinterpret_cast<uint4*>(&sm.x[sbl][plane][r][8 * c8]) = tmp[k];
        }
        sm.g[gs][gr][gq] = gv;
        sm.inv[is][ir] = iv;
    }
    __syncthreads();

    f4_t acc[RT][NBT];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // One superblock of RT tiles: acc += (dC C - / + dM Cm) / s
    auto compute = [&](int sbl, const Raw* r) {
        f4_t C[RT][NBT], Cm[RT][NBT];
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) C[t][bt] = Cm[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        float dC[RT], dM[RT];
        h8_t bm[RT];   // B operand of the group-sum MFMA (k = 8 s + e)
        if constexpr (kQ4) {
            uint32_t slo[RT][4], shi[RT][4];
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const uint4 h = r[t].hdr;
                dC[t] = half_lo(h.x) * 16384.0f;     // codes carry 2^-14
                dM[t] = half_hi(h.x) * 32.0f;        // group sums are staged / 32
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t sc0, m0, sc1, m1;
                    q4k_scale_min(h.y, h.z, h.w, 2 * j, sc0, m0);
                    q4k_scale_min(h.y, h.z, h.w, 2 * j + 1, sc1, m1);
                    slo[t][j] = h2dup((float)sc0 * 1024.0f);
                    shi[t][j] = h2dup((float)sc1 * 64.0f);
                    // minimum term: segments 0 (hi sums) and 1 (lo sums) hold group e; 2, 3 zero
                    bm[t][2 * j] = s < 2 ? (_Float16)(float)m0 : (_Float16)0.0f;
                    bm[t][2 * j + 1] = s < 2 ? (_Float16)(float)m1 : (_Float16)0.0f;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int kk = (2 * j + half) * 32 + 8 * s;
                    h8_t ah[NBT], al[NBT];
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt) {
                        ah[bt] = *reinterpret_cast<const h8_t*>(&sm.x[sbl][0][bt * 16 + li][kk]);
                        al[bt] = *reinterpret_cast<const h8_t*>(&sm.x[sbl][1][bt * 16 + li][kk]);
                    }
#pragma unroll
                    for (int t = 0; t < RT; ++t) {
                        const uint32_t w0 = r[t].q[j].x, w1 = r[t].q[j].y, v0 = w0 >> 8, v1 = w1 >> 8;
                        const uint32_t M = half ? 0x00F000F0u : 0x000F000Fu;
                        const uint32_t sp = half ? shi[t][j] : slo[t][j];
                        const uint4 q4 = {pk_mul_f16(w0 & M, sp), pk_mul_f16(v0 & M, sp), pk_mul_f16(w1 & M, sp),
                                          pk_mul_f16(v1 & M, sp)};
                        const h8_t bw = __builtin_bit_cast(h8_t, q4);
#pragma unroll
                        for (int bt = 0; bt < NBT; ++bt) {
                            C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[bt], bw, C[t][bt], 0, 0, 0);
                            C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[bt], bw, C[t][bt], 0, 0, 0);
                        }
                    }
                }
        } else {
            // chunk c = 32 values = half c/4, l = 32(c%4) + 8s + [0,8); scale index
            // 8h + 2(c%4) + s/2.  Offset term k = 8 s + e: group 8(s%2) + e.
            uint32_t A[RT][2][2], B[RT][2][2], H[RT][2][2], scw[RT][4];
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)r[t].d);
                dC[t] = d * 16384.0f;   // codes carry 2^-14
                dM[t] = d * 512.0f;     // -32 sc x: sums staged / 16
#pragma unroll
                for (int i = 0; i < 4; ++i) scw[t][i] = funnel(r[t].sc[i], r[t].sc[i + 1], r[t].mis);
#pragma unroll
                for (int e = 0; e < 8; ++e) {   // group 8 (s % 2) + e
                    const uint32_t word = (s & 1) ? scw[t][2 + (e >> 2)] : scw[t][e >> 2];
                    bm[t][e] = (_Float16)(float)(-(int)(int8_t)((word >> (8 * (e & 3))) & 255u));
                }
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        A[t][hh][i] = funnel(r[t].a[hh][i], r[t].a[hh][i + 1], r[t].mis);
                        B[t][hh][i] = funnel(r[t].b[hh][i], r[t].b[hh][i + 1], r[t].mis);
                        H[t][hh][i] = funnel(r[t].h[hh][i], r[t].h[hh][i + 1], r[t].mis);
                    }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int hh = c >> 2, q4 = c & 3, hs = 2 * q4;
                const int kk = c * 32 + 8 * s;
                h8_t ah[NBT], al[NBT];
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt) {
                    ah[bt] = *reinterpret_cast<const h8_t*>(&sm.x[sbl][0][bt * 16 + li][kk]);
                    al[bt] = *reinterpret_cast<const h8_t*>(&sm.x[sbl][1][bt * 16 + li][kk]);
                }
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    // scale 8 hh + 2 q4 + s/2: word 2 hh + q4/2, byte 2 (q4 % 2) + s/2
                    const uint32_t word = scw[t][2 * hh + (q4 >> 1)];
                    const float scf = (float)(int)(int8_t)((word >> (8 * (2 * (q4 & 1) + (s >> 1)))) & 255u);
                    const uint32_t sp = h2dup(scf * 256.0f);
                    uint32_t v[4];
#pragma unroll
                    for (int d2 = 0; d2 < 2; ++d2) {
                        const uint32_t run = (q4 & 1) ? B[t][hh][d2] : A[t][hh][d2];
                        // 4 c per byte: nibble at bits 2..5, the two high bits at 6..7
                        const uint32_t nb = (q4 >> 1) ? (run >> 2) : (run << 2);
                        const uint32_t code = (nb & 0x3C3C3C3Cu) | ((H[t][hh][d2] << (6 - hs)) & 0xC0C0C0C0u);
                        v[2 * d2] = pk_mul_f16(code & 0x00FF00FFu, sp);
                        v[2 * d2 + 1] = pk_mul_f16((code >> 8) & 0x00FF00FFu, sp);
                    }
                    const h8_t bw = __builtin_bit_cast(h8_t, uint4{v[0], v[1], v[2], v[3]});
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt) {
                        C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[bt], bw, C[t][bt], 0, 0, 0);
                        C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[bt], bw, C[t][bt], 0, 0, 0);
                    }
                }
            }
        }
        // group-sum MFMA: A operand rows were laid out by xprep_kernel per k segment
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            const h8_t am = sm.g[sbl][bt * 16 + li][s];
#pragma unroll
            for (int t = 0; t < RT; ++t) Cm[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bm[t], Cm[t][bt], 0, 0, 0);
        }
        // Q4_K: minimum enters with -dmin; Q6_K: the -sc sign is inside bm
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float inv = sm.inv[sbl][bt * 16 + 4 * s + e];
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    float v = dC[t] * C[t][bt][e];
                    v = kQ4 ? fmaf(-dM[t], Cm[t][bt][e], v) : fmaf(dM[t], Cm[t][bt][e], v);
                    acc[t][bt][e] = fmaf(v, inv, acc[t][bt][e]);
                }
            }
    };

    // Tile finished: epilogue (one slab) or partial sums [slab][batch][virtual row].
    auto finish = [&](int it) {
        const int tg = gw + (it / nsb) * nw;
        float tmax[NBT][4];
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int e = 0; e < 4; ++e) tmax[bt][e] = -INFINITY;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const int v = tg * kTile + t * 16 + li;
            const bool ok = v < total_rows;
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int b = bt * 16 + 4 * s + e;
                    const float val = acc[t][bt][e];
                    if (nslab > 1) {
                        if (ok && b < batch) part[((int64_t)slab * kMaxBatchTile + b) * total_rows + v] = val;
                    } else if constexpr (MODE == kSwiglu) {
                        const float up = dpp_mov<0xB1>(val);   // odd lane holds the up row
                        if (ok && b < batch && !(li & 1)) y[(int64_t)b * rows + (v >> 1)] = swiglu(val, up);
                    } else if constexpr (MODE == kAccumulate) {
                        if (ok && b < batch) y[(int64_t)b * rows + v] += val;
                    } else {
                        if (ok && b < batch) y[(int64_t)b * rows + v] = val;
                        if (ok) tmax[bt][e] = fmaxf(tmax[bt][e], val);
                    }
                    acc[t][bt][e] = 0.0f;
                }
        }
        if constexpr (MODE == kLogits) {
            if (nslab == 1) {   // per-tile maxima for the argmax: pmax[b][tg]
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float m = tmax[bt][e];
                        m = group_max(m, 16);
                        const int b = bt * 16 + 4 * s + e;
                        if (li == 0 && b < batch) pmax[(int64_t)b * ntg + tg] = m;
                    }
            }
        }
    };

    // Iteration it multiplies buffer it % DEPTH while it + DEPTH - 1 loads.
    for (int it0 = 0; it0 < nit; it0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int it = it0 + d;
            load_w(min(it + DEPTH - 1, nit - 1), buf[(d + DEPTH - 1) % DEPTH]);
            if (it < nit) {
                compute(it % nsb, buf[d]);
                if ((it + 1) % nsb == 0) finish(it);
            }
        }
    }
}

// Adds the K-slab partials in slab order and applies the epilogue.  In kSwiglu the
// virtual rows interleave gate (even) and up (odd).  kLogits also writes per-block
// maxima pmax[b * gridDim.x + block] for the argmax.
template <int MODE, int NS>
__global__ void __launch_bounds__(256) gemm_reduce_kernel(const float* __restrict__ part, int nslab, int rows,
                                                          int batch, float* __restrict__ y, float* __restrict__ pmax) {
    const int total_rows = MODE == kSwiglu ? 2 * rows : rows;
    const int b = blockIdx.y;
    const int r = blockIdx.x * 256 + threadIdx.x;
    float v = -INFINITY;
    if (r < rows && b < batch) {
        // every slab's value is loaded before the first add (see add_slabs)
        float s = 0.0f, s2 = 0.0f;
        const float* p0 = part + (int64_t)b * total_rows;
        const int64_t ks = (int64_t)kMaxBatchTile * total_rows;
        if constexpr (NS == 0) {
            for (int k = 0; k < nslab; ++k) {
                if constexpr (MODE == kSwiglu) {
                    const float2 gu = *reinterpret_cast<const float2*>(p0 + k * ks + 2 * r);
                    s += gu.x;
                    s2 += gu.y;
                } else {
                    s += p0[k * ks + r];
                }
            }
        } else if constexpr (MODE == kSwiglu) {
            float2 gu[NS];
#pragma unroll
            for (int k = 0; k < NS; ++k) gu[k] = *reinterpret_cast<const float2*>(p0 + min(k, nslab - 1) * ks + 2 * r);
#pragma unroll
            for (int k = 0; k < NS; ++k)
                if (k < nslab) {
                    s += gu[k].x;
                    s2 += gu[k].y;
                }
        } else {
            float t[NS];
#pragma unroll
            for (int k = 0; k < NS; ++k) t[k] = p0[min(k, nslab - 1) * ks + r];
#pragma unroll
            for (int k = 0; k < NS; ++k)
                if (k < nslab) s += t[k];
        }
        float* out = y + (int64_t)b * rows + r;
        if constexpr (MODE == kStore || MODE == kLogits) *out = s;
        else if constexpr (MODE == kAccumulate) *out += s;
        else *out = swiglu(s, s2);
        v = s;
    }
    if constexpr (MODE == kLogits) {
        v = wave_max_dpp(v);
        __shared__ float red[4];
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        if (threadIdx.x == 0 && b < batch)
            pmax[(int64_t)b * gridDim.x + blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
}

}  // namespace rta
