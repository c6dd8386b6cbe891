// rta_tiled.hpp -- packed ("tiled") K-quant weights and their matrix-core readout.
//
// The GGUF row layout spreads the 16 rows a matrix-core tile multiplies over 16
// separate blocks per superblock, so every load instruction touches 16 short
// pieces of as many cache lines, and each line is read piecewise by several
// instructions.  rta_pack rewrites a matrix once (at load time, same size) into
// tiles of 16 rows x 1 superblock whose bytes are laid out in the order the 64
// lanes of a wave consume them: every load instruction of the readout then reads
// whole contiguous lines that no other instruction needs.
//
//   Q4_K tile, 2304 bytes (16 x 144):
//     [0, 256)      row r's 16-byte block header at 16 r: d and dmin as in the GGUF
//                   block, then its eight 6-bit scales and minima regrouped per lane
//                   segment: bits [24 s, 24 s + 24) of the 96-bit little-endian field in
//                   bytes 4..15 hold sc(2 s), sc(2 s + 1), m(2 s), m(2 s + 1) at bit
//                   offsets 0, 6, 12, 18 (the groups lane segment s multiplies; one
//                   funnel shift and four field extracts decode them)
//     [256, 1280)   lane l = 16 s + r: bytes [32 s, 32 s + 16) of row r's 128 quant bytes
//     [1280, 2304)  lane l: bytes [32 s + 16, 32 s + 32)
//   Q6_K tile, 3360 bytes (16 x 210):
//     [0, 256)      row r's 16 int8 scales at 16 r
//     [256, 288)    row r's f16 d at 256 + 2 r
//     [288, 1312)   lane l = 16 s + r, h = s / 2, o = 16 (s % 2): ql[64 h + o, +16)
//     [1312, 2336)  lane l: ql[64 h + 32 + o, +16)
//     [2336, 3360)  lane l: qh[32 h + o, +16)
//   Tiles are ordered [row tile][superblock]; a last partial row tile is padded
//   with zero rows (d = 0: they contribute nothing and are never written).
//
// Lane (r, s) of a tile thus holds 64 of the superblock's 256 values, 8 per matrix
// core instruction m = 0..7, each 8 from one scale group:
//   Q4_K  columns 64 s + 8 m + [0, 8): low nibbles (group 2 s) for m < 4, high
//         nibbles (group 2 s + 1) for m >= 4
//   Q6_K  columns 128 (s/2) + 32 (m/2) + 16 (s%2) + 8 (m%2) + [0, 8): group
//         8 (s/2) + 2 (m/2) + s%2
// and x is read from LDS at exactly those columns (k-permuted inside each 8 as in
// the row-layout path).  The minimum (Q4_K) / -32 offset (Q6_K) terms use group
// sums of x that xprep_kernel lays out per lane segment to match.
#pragma once
#include "rta_gemm.hpp"
#include "rta_remap.hpp"

namespace rta {

constexpr int kTiled = 0x100;   // format flag: RTA_Q4_K | kTiled, RTA_Q6_K | kTiled

template <int FMT>
struct TileFmt;

template <>
struct TileFmt<RTA_Q4_K> {
    static constexpr int kBytes = 2304, kBlock = 144;
    struct Raw { uint4 hdr, q0, q1; };
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ c, int lane, Raw& r) {
        r.hdr = *reinterpret_cast<const uint4*>(c + 16 * (lane & 15));
        r.q0 = *reinterpret_cast<const uint4*>(c + 256 + 16 * lane);
        r.q1 = *reinterpret_cast<const uint4*>(c + 1280 + 16 * lane);
    }
    // Bytes 4..15 of a tile row header from the GGUF block's 12 scale bytes q (the
    // get_scale_min_k4 decoding of resident_quant.glsl:10-19): the 96-bit field of
    // the layout above, as three little-endian words.
    __host__ __device__ static inline void scale_field(const uint8_t* q, uint32_t f[3]) {
        uint64_t lo = 0, hi = 0;   // bits [0, 64), [64, 96)
        auto put = [](uint64_t& l, uint64_t& h, uint32_t v, int b) {   // 6-bit v at bit b
            if (b >= 64) {
                h |= (uint64_t)v << (b - 64);
            } else {
                l |= (uint64_t)v << b;
                if (b > 58) h |= (uint64_t)v >> (64 - b);   // straddles bit 64
            }
        };
        for (int g = 0; g < 8; ++g) {
            const int j = g & 3;
            const uint32_t sc = g < 4 ? (q[j] & 63u) : ((q[j + 8] & 15u) | ((q[j] >> 6) << 4));
            const uint32_t m = g < 4 ? (q[j + 4] & 63u) : ((q[j + 8] >> 4) | ((q[j + 4] >> 6) << 4));
            const int s = g >> 1, k = g & 1;
            const int bs = 24 * s + 6 * k, bm = bs + 12;   // bit offsets of sc(g), m(g)
            put(lo, hi, sc, bs);
            put(lo, hi, m, bm);
        }
        f[0] = (uint32_t)lo;
        f[1] = (uint32_t)(lo >> 32);
        f[2] = (uint32_t)hi;
    }
    // byte offset, inside row r's GGUF block, of tile byte o (o even), or -1 for the
    // regrouped scale bytes (header bytes 4..15, see scale_field)
    __host__ __device__ static inline int source(int o, int& r) {
        if (o < 256) { r = o >> 4; return (o & 15) < 4 ? (o & 15) : -1; }
        const int k = o < 1280 ? 0 : 1, p = o - (k ? 1280 : 256), l = p >> 4;
        r = l & 15;
        return 16 + 32 * (l >> 4) + 16 * k + (p & 15);
    }
};

template <>
struct TileFmt<RTA_Q6_K> {
    static constexpr int kBytes = 3360, kBlock = 210;
    struct Raw { uint4 sc, a, b, h; uint32_t d; };
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ c, int lane, Raw& r) {
        r.sc = *reinterpret_cast<const uint4*>(c + 16 * (lane & 15));
        r.d = *reinterpret_cast<const uint16_t*>(c + 256 + 2 * (lane & 15));
        r.a = *reinterpret_cast<const uint4*>(c + 288 + 16 * lane);
        r.b = *reinterpret_cast<const uint4*>(c + 1312 + 16 * lane);
        r.h = *reinterpret_cast<const uint4*>(c + 2336 + 16 * lane);
    }
    __host__ __device__ static inline int source(int o, int& r) {
        if (o < 256) { r = o >> 4; return 192 + (o & 15); }
        if (o < 288) { r = (o - 256) >> 1; return 208 + (o & 1); }
        const int k = o < 1312 ? 0 : o < 2336 ? 1 : 2;
        const int p = o - (k == 0 ? 288 : k == 1 ? 1312 : 2336), l = p >> 4, s = l >> 4;
        r = l & 15;
        const int h = s >> 1, ofs = 16 * (s & 1) + (p & 15);
        return k == 0 ? 64 * h + ofs : k == 1 ? 64 * h + 32 + ofs : 128 + 32 * h + ofs;
    }
};

// One thread per 2 bytes of the packed matrix; tile row r holds GGUF row m.source_row(r).
template <int FMT>
__global__ void __launch_bounds__(256) pack_kernel(const uint8_t* __restrict__ src, int rows, int cols,
                                                   uint8_t* __restrict__ dst, int64_t n2, const Remap m) {
    using F = TileFmt<FMT>;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n2) return;
    const int64_t o = 2 * i;
    const int nsb = cols >> 8;
    const int64_t chunk = o / F::kBytes;
    const int within = (int)(o - chunk * F::kBytes);
    const int64_t tile = chunk / nsb;
    const int sb = (int)(chunk - tile * nsb);
    int r;
    const int off = F::source(within, r);
    const int64_t row = tile * 16 + r;
    uint16_t v = 0;
    if (row < rows) {
        const uint8_t* blk = src + m.source_row(row) * (int64_t)nsb * F::kBlock + (int64_t)sb * F::kBlock;
        if constexpr (FMT == RTA_Q4_K) {
            if (off < 0) {   // regrouped scale bytes: half-word (within - 4) / 2 of the field
                uint32_t f[3];
                F::scale_field(blk + 4, f);
                const int h = (within & 15) - 4;   // 0, 2, .., 10
                v = (uint16_t)(f[h >> 2] >> (8 * (h & 3)));
            } else {
                v = (uint16_t)(blk[off] | (blk[off + 1] << 8));
            }
        } else {
            v = (uint16_t)(blk[off] | (blk[off + 1] << 8));
        }
    }
    *reinterpret_cast<uint16_t*>(dst + o) = v;
}


__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Scales and minima of groups 2 s and 2 s + 1 from a packed Q4_K tile row header h (the
// regrouped field of TileFmt<RTA_Q4_K>): the words holding segment s's 24 bits are
// picked with the lane's masks (bit selects: an indexed pick among the header's words
// would go through memory), one funnel shift brings the bits down, four field extracts
// split them.
// Waves w and w + 4 of an 8-wave workgroup share a SIMD, whose arbiter issues for the
// older wave first: left to it, the older wave finishes its items ~3 us before the
// younger one, which then runs alone on the SIMD.  The two take turns at the higher
// issue priority, item by item (it: the wave's item index), and finish together.
__device__ __forceinline__ void take_turns(int wave, int it) {
    if (((wave >> 2) ^ it) & 1)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(0);
}

struct Q4kSegment {
    uint32_t m01, m2, shift;   // all-ones for segments 0-1, for segment 2; 24 s mod 32
    __device__ explicit Q4kSegment(int s)
        : m01(s < 2 ? ~0u : 0u), m2(s == 2 ? ~0u : 0u), shift((uint32_t)(24 * s) & 31u) {}
};
__device__ __forceinline__ void q4k_tile_scale_min(const uint4& h, const Q4kSegment& g, uint32_t& sc0, uint32_t& sc1,
                                                   uint32_t& m0, uint32_t& m1) {
    const uint32_t w23 = (h.z & g.m2) | (h.w & ~g.m2);      // segment 2: z, segment 3: w
    const uint32_t lo = (h.y & g.m01) | (w23 & ~g.m01);
    const uint32_t hi = (h.z & g.m01) | (h.w & ~g.m01);
    const uint32_t f = __builtin_amdgcn_alignbit(hi, lo, g.shift);
    sc0 = f & 63u;
    sc1 = (f >> 6) & 63u;
    m0 = (f >> 12) & 63u;
    m1 = (f >> 18) & 63u;
}

// (f16(v), f16(v)) for an integer v < 2^11 times a power of two c (exact in binary16)
__device__ __forceinline__ uint32_t h2dup_scaled(uint32_t v, float c) {
    const float x = (float)v * c;
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, x));
}

// Prepares x rows [0, 16 NBT) over superblocks [sb0, sb0 + nsb) straight into LDS,
// in the tiled-readout layouts (kXpQ4Tile / kXpQ6Tile of xprep_kernel): per (row,
// superblock) a power-of-two scale s with max|x s| in [2^13, 2^14), x s as binary16
// hi + lo (k-permuted inside each 8-value segment), the group sums of x s (/32 for
// Q4_K, /16 for Q6_K) as hi + lo, and 1/s (0 for rows >= batch).  32 threads per
// (row, superblock), 8 columns each.  load() issues every x load; store() (after the
// weight prefetch has been issued behind them) prepares and writes LDS.
template <int FMT, int NBT>
struct XStage {
    using Smem = GemmSmem<NBT>;
    static constexpr int kRows = Smem::kRows;
    static constexpr int kGroups = 64 * kGemmWaves / 32;            // (row, superblock) pairs per round
    static constexpr int kRounds = Smem::kSb * kRows / kGroups;
    float v[kRounds][8];
    float4 rnp[kRounds];   // deferred-norm sums of the round's row

    __device__ __forceinline__ void load(const float* __restrict__ x, int cols, int batch, int sb0, int nsb,
                                         const RowNorm& rn) {
        const int grp = threadIdx.x >> 5, t = threadIdx.x & 31;
        const int npairs = nsb * kRows;                           // a multiple of kGroups
#pragma unroll
        for (int k = 0; k < kRounds; ++k) {
            const int pr = grp + k * kGroups, sbl = pr / kRows, r = pr - sbl * kRows;
            // unconditional (x's first float4 stands in when there is no deferred norm):
            // a guarded load would wait on the spot
            rnp[k] = rn.part ? rn.part[r < batch ? r : batch - 1] : *reinterpret_cast<const float4*>(x);
            if (pr < npairs && r < batch) {
                const float4* src =
                    reinterpret_cast<const float4*>(x + (int64_t)r * cols + (int64_t)(sb0 + sbl) * 256 + 8 * t);
                const float4 a = src[0], c = src[1];
                v[k][0] = a.x; v[k][1] = a.y; v[k][2] = a.z; v[k][3] = a.w;
                v[k][4] = c.x; v[k][5] = c.y; v[k][6] = c.z; v[k][7] = c.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = 0.0f;
            }
        }
    }

    __device__ __forceinline__ void store(Smem& sm, int batch, int nsb, const RowNorm& rn) const {
        const int grp = threadIdx.x >> 5, t = threadIdx.x & 31;
        const int npairs = nsb * kRows;
#pragma unroll
        for (int k = 0; k < kRounds; ++k) {
            const int pr = grp + k * kGroups, sbl = pr / kRows, r = pr - sbl * kRows;
            if (pr >= npairs) break;                              // uniform over the workgroup
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[k][i]));
            m = group_max(m, 32);   // within 32 lanes
            const int e = operand_exponent(m);
            const float sc = ldexpf(1.0f, 14 - e);
            if (t == 0) {
                const float f = rn.part ? row_norm_factor(rn, rnp[k]) : 1.0f;
                sm.inv[sbl][r] = r < batch ? ldexpf(1.0f, e - 14) * f : 0.0f;
            }
            constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
            _Float16 hi[8], lo[8];
            float sum8 = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float w = v[k][perm[i]] * sc;
                hi[i] = (_Float16)w;
                lo[i] = (_Float16)(w - (float)hi[i]);
                sum8 += v[k][i] * sc;
            }
            *reinterpret_cast<h8_t*>(&sm.x[sbl][0][r][8 * t]) = h8_t{hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6], hi[7]};
            *reinterpret_cast<h8_t*>(&sm.x[sbl][1][r][8 * t]) = h8_t{lo[0], lo[1], lo[2], lo[3], lo[4], lo[5], lo[6], lo[7]};
            _Float16* g = reinterpret_cast<_Float16*>(&sm.g[sbl][r][0]);   // 4 segments x 8
            const float s16 = sum8 + dpp_mov<0xB1>(sum8);
            const float s32 = s16 + dpp_mov<0x4E>(s16);
            if constexpr (FMT == RTA_Q6_K) {
                if ((t & 1) == 0) {   // 16-group u = 8 hh + 2 q + sg -> segment 2 hh + sg, slot 2 q
                    const int u = t >> 1;
                    const float w = s16 * (1.0f / 16.0f);
                    const _Float16 h = (_Float16)w, l = (_Float16)(w - (float)h);
                    const int seg = 2 * (u >> 3) + (u & 1), q = (u >> 1) & 3;
                    g[8 * seg + 2 * q] = h;
                    g[8 * seg + 2 * q + 1] = l;
                }
            } else {
                const int q = t >> 2;  // 32-group: segment q / 2, slots 2 (q % 2), +1; zeros at +4, +5
                if ((t & 3) == 0) {
                    const float w = s32 * (1.0f / 32.0f);
                    const _Float16 h = (_Float16)w, l = (_Float16)(w - (float)h);
                    g[8 * (q >> 1) + 2 * (q & 1)] = h;
                    g[8 * (q >> 1) + 2 * (q & 1) + 1] = l;
                } else if ((t & 3) == 1) {
                    g[8 * (q >> 1) + 4 + 2 * (q & 1)] = (_Float16)0.0f;
                    g[8 * (q >> 1) + 5 + 2 * (q & 1)] = (_Float16)0.0f;
                }
            }
        }
    }
};

// Units of work: pairs of 16-row tiles (t = 0, 1).  In kSwiglu the pair is (gate
// tile T, up tile T) of one unit T; otherwise tiles (a + 2u, a + 2u + 1) of the
// wave's contiguous tile range [a, b), the second one absent at an odd end.
template <int FMT, int NBT, int MODE>
__global__ void __launch_bounds__(64 * kGemmWaves) gemm_tiled_kernel(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, const int rows, const int cols,
    const float* __restrict__ x, const int batch, float* __restrict__ y, float* __restrict__ part,
    float* __restrict__ pmax, const int sb_per_slab, const int wgs_per_slab, const RowNorm rn) {
    constexpr bool kQ4 = FMT == RTA_Q4_K;
    using F = TileFmt<FMT>;
    using Raw = typename F::Raw;
    using Smem = GemmSmem<NBT>;
    __shared__ Smem sm;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slab = blockIdx.y, pos = blockIdx.x;   // grid (wgs_per_slab, slabs)
    const int nslab = gridDim.y;
    const int nsbt = cols >> 8;
    const int sb0 = slab * sb_per_slab;
    const int nsb = min(sb_per_slab, nsbt - sb0);

    // x loads first (vector-memory loads complete in order, so the x slab is not held
    // up behind the weights; and a kernel starts with cold instruction and scalar
    // caches, so nothing is worked out ahead of them that they do not need), then
    // DEPTH - 1 superblocks of weights, then the x prep.
    XStage<FMT, NBT> xs;
    xs.load(x, cols, batch, sb0, nsb, rn);

    const int s = lane >> 4, li = lane & 15;
    const Q4kSegment seg(s);
    const int total_rows = MODE == kSwiglu ? 2 * rows : rows;
    const int ntile = (rows + 15) >> 4;

    // ---- balanced contiguous tile range of this wave: floor(g ntile / nw) in 32 bits,
    // g (q nw + r) / nw = g q + floor(g r / nw) with g r < nw^2
    const int gw = pos * kGemmWaves + wave, nw = wgs_per_slab * kGemmWaves;
    const int tq = ntile / nw, tr = ntile - tq * nw;
    const int ta = gw * tq + gw * tr / nw, tb = (gw + 1) * tq + (gw + 1) * tr / nw;
    const int nunit = MODE == kSwiglu ? tb - ta : (tb - ta + 1) >> 1;
    const int nit = nunit * nsb;

    auto tiles_of = [&](int u, int& t0, int& t1) {
        if constexpr (MODE == kSwiglu) { t0 = t1 = ta + u; }
        else { t0 = ta + 2 * u; t1 = min(t0 + 1, tb - 1); }
    };
    // (unit, superblock) of the next weight load, advanced one iteration at a time and
    // held at the last iteration (no division in the loop)
    int lu = 0, lsb = 0, lit = 0;
    auto load_next = [&](Raw* dst) {
        int t0, t1;
        tiles_of(lu, t0, t1);
        const int64_t sb = sb0 + lsb;
        F::load(w + ((int64_t)t0 * nsbt + sb) * F::kBytes, lane, dst[0]);
        F::load((MODE == kSwiglu ? w2 : w) + ((int64_t)t1 * nsbt + sb) * F::kBytes, lane, dst[1]);
        if (lit < nit - 1) {
            ++lit;
            if (++lsb == nsb) {
                lsb = 0;
                ++lu;
            }
        }
    };

    constexpr int DEPTH = 2;   // one superblock loads while the current one multiplies
    Raw buf[DEPTH][2];
    if (nit > 0) {
#pragma unroll
        for (int d = 0; d < DEPTH - 1; ++d) load_next(buf[d]);
    }
    xs.store(sm, batch, nsb, rn);
    __syncthreads();

    f4_t acc[2][NBT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // One superblock of the unit's tiles (the second only when has2).
    // One superblock of the unit's two tiles.  Both tiles are always multiplied (at an
    // odd end of the wave's range the second repeats the first and finish() skips it),
    // so the loop body has no branches and the x operands of the next column offset
    // can be read while the current MFMAs run.  Per column offset the eight MFMAs go
    // hi planes first, then lo planes, so an accumulator's two MFMAs are four apart.
    auto compute = [&](int sbl, const Raw* r) {
        f4_t C[2][NBT], Cm[2][NBT];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) C[t][bt] = Cm[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        float dC[2], dM[2];
        h8_t bm[2];
        // x operands of column offset kk, read once and used by both tiles
        auto xload = [&](int kk, h8_t* ah, h8_t* al) {
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                ah[bt] = *reinterpret_cast<const h8_t*>(&sm.x[sbl][0][bt * 16 + li][kk]);
                al[bt] = *reinterpret_cast<const h8_t*>(&sm.x[sbl][1][bt * 16 + li][kk]);
            }
        };
        auto mma8 = [&](const h8_t* ah, const h8_t* al, const h8_t* bw) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt)
                    C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[bt], bw[t], C[t][bt], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt)
                    C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[bt], bw[t], C[t][bt], 0, 0, 0);
        };
        if constexpr (kQ4) {
            uint32_t slo[2], shi[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint4 h = r[t].hdr;
                dC[t] = half_lo(h.x) * 16384.0f;     // codes carry 2^-14
                dM[t] = half_hi(h.x) * 32.0f;        // group sums are staged / 32
                uint32_t sc0, m0, sc1, m1;
                q4k_tile_scale_min(h, seg, sc0, sc1, m0, m1);
                slo[t] = h2dup_scaled(sc0, 1024.0f);
                shi[t] = h2dup_scaled(sc1, 64.0f);
                bm[t] = __builtin_bit_cast(h8_t, uint4{h2dup_scaled(m0, 1.0f), h2dup_scaled(m1, 1.0f), 0u, 0u});
            }
            h8_t ah[NBT], al[NBT];
            xload(64 * s, ah, al);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                h8_t bw[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int mq = m & 3;
                    const uint32_t w0 = word_of(mq < 2 ? r[t].q0 : r[t].q1, 2 * (mq & 1));
                    const uint32_t w1 = word_of(mq < 2 ? r[t].q0 : r[t].q1, 2 * (mq & 1) + 1);
                    const uint32_t M = m < 4 ? 0x000F000Fu : 0x00F000F0u;
                    const uint32_t sp = m < 4 ? slo[t] : shi[t];
                    const uint4 q4 = {pk_mul_f16(w0 & M, sp), pk_mul_f16((w0 >> 8) & M, sp), pk_mul_f16(w1 & M, sp),
                                      pk_mul_f16((w1 >> 8) & M, sp)};
                    bw[t] = __builtin_bit_cast(h8_t, q4);
                }
                h8_t nh[NBT], nl[NBT];
                if (m < 7) xload(64 * s + 8 * (m + 1), nh, nl);
                mma8(ah, al, bw);
                if (m < 7) {
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt) {
                        ah[bt] = nh[bt];
                        al[bt] = nl[bt];
                    }
                }
            }
        } else {
            const int hh = s >> 1, sg = s & 1;
            float scq[2][4];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)r[t].d);
                dC[t] = d * 16384.0f;   // codes carry 2^-14
                dM[t] = d * 512.0f;     // -32 sc x: sums staged / 16
                // scales of groups 8 hh + 2 q + sg, q = 0..3: words 2 hh (q < 2) and 2 hh + 1
                const uint32_t wa = hh ? r[t].sc.z : r[t].sc.x, wb = hh ? r[t].sc.w : r[t].sc.y;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    scq[t][q] = (float)(int)(int8_t)(((q < 2 ? wa : wb) >> (8 * (2 * (q & 1) + sg))) & 255u);
                bm[t] = h8_t{(_Float16)-scq[t][0], (_Float16)-scq[t][0], (_Float16)-scq[t][1], (_Float16)-scq[t][1],
                             (_Float16)-scq[t][2], (_Float16)-scq[t][2], (_Float16)-scq[t][3], (_Float16)-scq[t][3]};
            }
            auto col = [&](int m) { return 128 * hh + 32 * (m >> 1) + 16 * sg + 8 * (m & 1); };
            h8_t ah[NBT], al[NBT];
            xload(col(0), ah, al);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const int q = m >> 1, half = m & 1;
                h8_t bw[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint4& run = (q & 1) ? r[t].b : r[t].a;
                    const uint32_t sp = h2dup(scq[t][q] * 256.0f);
                    uint32_t v[4];
#pragma unroll
                    for (int d2 = 0; d2 < 2; ++d2) {
                        const uint32_t rw = word_of(run, 2 * half + d2), hw = word_of(r[t].h, 2 * half + d2);
                        // 4 c per byte: nibble at bits 2..5, the two high bits at 6..7
                        const uint32_t nb = (q >> 1) ? (rw >> 2) : (rw << 2);
                        const uint32_t code = (nb & 0x3C3C3C3Cu) | ((hw << (6 - 2 * q)) & 0xC0C0C0C0u);
                        v[2 * d2] = pk_mul_f16(code & 0x00FF00FFu, sp);
                        v[2 * d2 + 1] = pk_mul_f16((code >> 8) & 0x00FF00FFu, sp);
                    }
                    bw[t] = __builtin_bit_cast(h8_t, uint4{v[0], v[1], v[2], v[3]});
                }
                h8_t nh[NBT], nl[NBT];
                if (m < 7) xload(col(m + 1), nh, nl);
                mma8(ah, al, bw);
                if (m < 7) {
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt) {
                        ah[bt] = nh[bt];
                        al[bt] = nl[bt];
                    }
                }
            }
        }
        // group-sum MFMA (A operand laid out per lane segment by the x staging)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            const h8_t am = sm.g[sbl][bt * 16 + li][s];
            Cm[0][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bm[0], Cm[0][bt], 0, 0, 0);
            Cm[1][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bm[1], Cm[1][bt], 0, 0, 0);
        }
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float inv = sm.inv[sbl][bt * 16 + 4 * s + e];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    float v = dC[t] * C[t][bt][e];
                    v = kQ4 ? fmaf(-dM[t], Cm[t][bt][e], v) : fmaf(dM[t], Cm[t][bt][e], v);
                    acc[t][bt][e] = fmaf(v, inv, acc[t][bt][e]);
                }
            }
    };

    // Unit finished: epilogue (one slab) or partial sums [slab][batch][virtual row].
    auto finish = [&](int u) {
        int t0, t1;
        tiles_of(u, t0, t1);
        const bool has2 = MODE == kSwiglu || t1 != t0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (t == 1 && !has2) break;
            const int row = 16 * (t == 0 ? t0 : t1) + li;
            const bool ok = row < rows;
            float tmax[NBT][4];
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int b = bt * 16 + 4 * s + e;
                    const float val = acc[t][bt][e];
                    tmax[bt][e] = ok ? val : -INFINITY;
                    if (nslab > 1) {
                        const int v = MODE == kSwiglu ? 2 * row + t : row;
                        if (ok && b < batch) part[((int64_t)slab * kMaxBatchTile + b) * total_rows + v] = val;
                    } else if constexpr (MODE == kSwiglu) {
                        if (t == 1 && ok && b < batch) y[(int64_t)b * rows + row] = swiglu(acc[0][bt][e], val);
                    } else if constexpr (MODE == kAccumulate) {
                        if (ok && b < batch) y[(int64_t)b * rows + row] += val;
                    } else {
                        if (ok && b < batch) y[(int64_t)b * rows + row] = val;
                    }
                }
            if constexpr (MODE == kLogits) {
                if (nslab == 1) {   // per-tile maxima for the argmax: pmax[b][tile]
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float m = tmax[bt][e];
                            m = group_max(m, 16);
                            const int b = bt * 16 + 4 * s + e;
                            if (li == 0 && b < batch) pmax[(int64_t)b * ntile + (t == 0 ? t0 : t1)] = m;
                        }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    };

    int cu = 0, csb = 0;   // (unit, superblock) being multiplied
    for (int it0 = 0; it0 < nit; it0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int it = it0 + d;
            load_next(buf[(d + DEPTH - 1) % DEPTH]);
            if (it < nit) {
                take_turns(wave, it);
                compute(csb, buf[d]);
                if (csb == nsb - 1) finish(cu);
                if (++csb == nsb) {
                    csb = 0;
                    ++cu;
                }
            }
        }
    }
}

}  // namespace rta
