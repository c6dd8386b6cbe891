// rta_packed.hpp -- the packed-tile readout of a decode step whose x arrives already
// in the matrix-core layout.
//
// residual_norm_image_kernel (the residual add and RMSNorm in front of the in- and
// gate/up projections) writes x = hidden * w as one image per superblock, laid out
// exactly as the readout keeps it in LDS:
//   x[2][rows][kXStride]  x s as binary16 hi and lo (k-permuted inside each 8),
//                         s a power of two per (row, superblock), max|x s| in [2^13, 2^14)
//   g[rows][4]            the group sums of x s (Q4_K /32, Q6_K /16) as hi + lo, laid
//                         out per lane segment of the tile format
//   inv[rows]             1 / s (0 past batch)
// and the row's sums of squares; the readout applies the row's RMSNorm factor
// 1 / sqrt(mean(hidden^2) + eps) to its results.  No workgroup of the readout converts
// x again (gemm_tiled_kernel converts its whole K slab in every workgroup).
//
// gemm_packed_kernel: one workgroup per compute unit and K slab; each wave takes a
// balanced contiguous range of units of TPW tiles (kSwiglu: TPW/2 gate tiles and the
// TPW/2 up tiles of the same rows) and, per superblock, reads the x operands of a
// column offset from LDS once for all TPW tiles.  The weights of the next DEPTH - 1
// superblocks are in flight in registers while one is multiplied.  The slab's images
// reach LDS by direct global -> LDS loads (global_load_lds_dwordx4).  Tile format and
// operand layouts are those of rta_tiled.hpp.
#pragma once
#include "rta_tiled.hpp"

namespace rta {

template <int NBT>
struct XImage {
    static constexpr int kRows = 16 * NBT;
    _Float16 x[2][kRows][kXStride];
    h8_t g[kRows][4];
    float inv[kRows];
};
static_assert(sizeof(XImage<1>) % 16 == 0 && sizeof(XImage<2>) % 16 == 0, "16-byte copies");

constexpr int kLdsBytes = 160 * 1024;
// superblocks of x one workgroup holds (its K slab)
template <int NBT>
constexpr int slab_capacity() {
    return (int)(kLdsBytes / sizeof(XImage<NBT>)) < 8 ? (int)(kLdsBytes / sizeof(XImage<NBT>)) : 8;
}

// Row b of one superblock image from the wave's 64 x 4 values v (lane l: columns 4 l ..
// 4 l + 3 of the superblock; zeros for a row past the batch, live false): scale, hi / lo
// planes, group sums and 1 / s, in the layout described at the top of this file.
template <int FMT, int NBT>
__device__ __forceinline__ void image_row(XImage<NBT>& im, int b, bool live, float4 v, int lane) {
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = wave_max_dpp(m);
    const int e = operand_exponent(m);
    const float sc = live ? ldexpf(1.0f, 14 - e) : 0.0f;
    if (lane == 0) im.inv[b] = live ? ldexpf(1.0f, e - 14) : 0.0f;
    // stored order inside each 8 columns: 0 2 1 3 4 6 5 7, i.e. (x, z, y, w) per float4
    const float t[4] = {v.x * sc, v.z * sc, v.y * sc, v.w * sc};
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        hi[k] = (_Float16)t[k];
        lo[k] = (_Float16)(t[k] - (float)hi[k]);
    }
    using h4 = _Float16 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4*>(&im.x[0][b][4 * lane]) = h4{hi[0], hi[1], hi[2], hi[3]};
    *reinterpret_cast<h4*>(&im.x[1][b][4 * lane]) = h4{lo[0], lo[1], lo[2], lo[3]};
    const float s4 = (t[0] + t[1]) + (t[2] + t[3]);
    // (DPP quad_perm xor 1, xor 2, then row_half_mirror, which for a quad-uniform value
    // reads the same partner value as xor 4)
    const float s8 = s4 + dpp_mov<0xB1>(s4);
    const float s16 = s8 + dpp_mov<0x4E>(s8);
    _Float16* g = reinterpret_cast<_Float16*>(&im.g[b][0]);   // 4 segments x 8
    if constexpr (FMT == RTA_Q6_K) {
        if ((lane & 3) == 0) {   // 16-group u = 8 hh + 2 q + sg -> segment 2 hh + sg, slot 2 q
            const int u = lane >> 2;
            const float wv = s16 * (1.0f / 16.0f);
            const _Float16 h = (_Float16)wv, l = (_Float16)(wv - (float)h);
            const int seg = 2 * (u >> 3) + (u & 1), q = (u >> 1) & 3;
            g[8 * seg + 2 * q] = h;
            g[8 * seg + 2 * q + 1] = l;
        }
    } else {
        const float s32 = s16 + dpp_mov<0x141>(s16);
        const int q = lane >> 3;   // 32-group: segment q / 2, slots 2 (q % 2), +1; zeros at +4, +5
        if ((lane & 7) == 0) {
            const float wv = s32 * (1.0f / 32.0f);
            const _Float16 h = (_Float16)wv, l = (_Float16)(wv - (float)h);
            g[8 * (q >> 1) + 2 * (q & 1)] = h;
            g[8 * (q >> 1) + 2 * (q & 1) + 1] = l;
        } else if ((lane & 7) == 1) {
            g[8 * (q >> 1) + 4 + 2 * (q & 1)] = (_Float16)0.0f;
            g[8 * (q >> 1) + 5 + 2 * (q & 1)] = (_Float16)0.0f;
        }
    }
}

// Block (column chunk c of 1024, row b), 256 threads, thread = 4 columns; wave k of
// the block = superblock 4c + k.  Rows b >= batch (up to the image's 16 NBT rows) write
// zeros.  For b < batch: hidden[b] += the K-slab partials [slab][32][width] (slab order)
// and ss[4 b + c] = the chunk's sum of hidden^2 (entries past the chunks zero), as
// residual_norm_deferred_kernel; out (may be null) = hidden * w in fp32 as well.
// NS: the slab loads in flight, NS >= nslab (1, 2, 4, 8, 16; every slab's load issued at
// once, indexes past the last slab clamped to it and not added), or 0 for a loop over more
// than 16 slabs.  The partials are added in slab order either way.
template <int FMT, int NBT, int NS>
__global__ void __launch_bounds__(256) residual_norm_image_kernel(float* __restrict__ hidden,
                                                                  const float* __restrict__ part, int nslab,
                                                                  const float* __restrict__ w, int width, int batch,
                                                                  float* __restrict__ ss, float* __restrict__ out,
                                                                  XImage<NBT>* __restrict__ img) {
    __shared__ float red[4];
    const int c = blockIdx.x, b = blockIdx.y, lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sb = 4 * c + wave, nsbt = width >> 8;
    const bool live = b < batch;   // uniform
    const int i = c * 256 + threadIdx.x;   // float4 of the row
    float4 v = float4{0.0f, 0.0f, 0.0f, 0.0f};
    float sq = 0.0f;
    if (live && sb < nsbt) {
        float4* hr = reinterpret_cast<float4*>(hidden + (int64_t)b * width);
        v = hr[i];
        if (nslab > 0) {   // uniform
            const float4* pr = reinterpret_cast<const float4*>(part + (int64_t)b * width) + i;
            const int64_t ps = (int64_t)32 * width / 4;   // float4s from one slab to the next
            if constexpr (NS > 0) {
                float4 p[NS];
#pragma unroll
                for (int k = 0; k < NS; ++k) p[k] = pr[(k < nslab ? k : nslab - 1) * ps];
#pragma unroll
                for (int k = 0; k < NS; ++k)
                    if (k < nslab) {
                        v.x += p[k].x;
                        v.y += p[k].y;
                        v.z += p[k].z;
                        v.w += p[k].w;
                    }
            } else {
#pragma unroll 4
                for (int k = 0; k < nslab; ++k) {
                    const float4 p = pr[k * ps];
                    v.x += p.x;
                    v.y += p.y;
                    v.z += p.z;
                    v.w += p.w;
                }
            }
            hr[i] = v;
        }
        sq = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        const float4 g = reinterpret_cast<const float4*>(w)[i];
        v = float4{v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w};
        if (out) reinterpret_cast<float4*>(out + (int64_t)b * width)[i] = v;
    }
    if (live) {
        // the block sum over every thread (threads past the row hold 0)
        sq = wave_sum_dpp(sq);
        if (lane == 0) red[wave] = sq;
        __syncthreads();
        if (threadIdx.x == 0) {
            ss[4 * b + c] = (red[0] + red[1]) + (red[2] + red[3]);
            if (c == 0)
                for (int z = gridDim.x; z < 4; ++z) ss[4 * b + z] = 0.0f;
        }
    }
    if (sb >= nsbt) return;   // uniform per wave
    image_row<FMT, NBT>(img[sb], b, live, v, lane);
}

// The SwiGLU of the gate/up K-slab partials [slab][32][2 rows] (gate at 2 r, up at 2 r + 1,
// added in slab order as gemm_reduce_kernel adds them) written as the x image of the down
// projection: block (c, b) as residual_norm_image_kernel, wave k = superblock 4 c + k of
// row b (zeros past the batch), lane = 4 consecutive columns.
// NS as in residual_norm_image_kernel.
template <int FMT, int NBT, int NS>
__global__ void __launch_bounds__(256) swiglu_image_kernel(const float* __restrict__ part, int nslab, int width,
                                                           int batch, XImage<NBT>* __restrict__ img) {
    const int c = blockIdx.x, b = blockIdx.y, lane = threadIdx.x & 63;
    const int sb = 4 * c + (threadIdx.x >> 6), nsbt = width >> 8;
    if (sb >= nsbt) return;   // uniform per wave
    const bool live = b < batch;   // uniform
    float4 v = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
        const int i = c * 256 + threadIdx.x;   // columns 4 i .. 4 i + 3
        float g[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float4* pr = reinterpret_cast<const float4*>(part + (int64_t)b * 2 * width) + 2 * i;
        const int64_t ps = (int64_t)32 * 2 * width / 4;   // float4s from one slab to the next
        auto add = [&](float4 a, float4 e) {
            g[0] += a.x;
            u[0] += a.y;
            g[1] += a.z;
            u[1] += a.w;
            g[2] += e.x;
            u[2] += e.y;
            g[3] += e.z;
            u[3] += e.w;
        };
        if constexpr (NS > 0) {
            float4 a[NS], e[NS];
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                const float4* p = pr + (k < nslab ? k : nslab - 1) * ps;
                a[k] = p[0];
                e[k] = p[1];
            }
#pragma unroll
            for (int k = 0; k < NS; ++k)
                if (k < nslab) add(a[k], e[k]);
        } else {
            for (int k = 0; k < nslab; ++k) add(pr[k * ps], pr[k * ps + 1]);
        }
        v = float4{swiglu(g[0], u[0]), swiglu(g[1], u[1]), swiglu(g[2], u[2]), swiglu(g[3], u[3])};
    }
    image_row<FMT, NBT>(img[sb], b, live, v, lane);
}

template <int FMT, int NBT, int MODE, int TPW, int NWAVES, int DEPTH>
__global__ void __launch_bounds__(64 * NWAVES) gemm_packed_kernel(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, const int rows, const int cols,
    const XImage<NBT>* __restrict__ xi, const int batch, float* __restrict__ y, float* __restrict__ part,
    const int sb_per_slab, const int wgs_per_slab, const RowNorm rn) {
    constexpr bool kQ4 = FMT == RTA_Q4_K;
    constexpr bool kDual = MODE == kSwiglu;
    static_assert(!kDual || TPW % 2 == 0, "SwiGLU units pair gate and up tiles");
    static_assert(MODE != kLogits, "the LM head runs on gemm_tiled_kernel");
    constexpr int kCap = slab_capacity<NBT>();
    using F = TileFmt<FMT>;
    using Raw = typename F::Raw;
    using Img = XImage<NBT>;
    __shared__ __align__(16) Img sx[kCap];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slab = blockIdx.y, pos = blockIdx.x;   // grid (wgs_per_slab, slabs)
    const int nslab = gridDim.y;
    const int nsbt = cols >> 8;
    const int sb0 = slab * sb_per_slab;
    const int nsb = min(sb_per_slab, nsbt - sb0);

    // The slab's x images go to LDS first, by direct global -> LDS loads (lane l of a
    // wave's instruction lands at the wave's LDS base + 16 l, so a wave moves 64
    // consecutive 16-byte words per instruction without a register round trip); all of
    // them are in flight at once, with DEPTH - 1 superblocks of weights issued behind
    // them.  They are issued before the work split is worked out: a kernel starts with
    // cold instruction and scalar caches, and the loads are the long pole.
    constexpr int kThreads = 64 * NWAVES;
    constexpr int kPer = (kCap * (int)(sizeof(Img) / 16) + kThreads - 1) / kThreads;
    const int n16 = nsb * (int)(sizeof(Img) / 16);
    const uint4* xsrc = reinterpret_cast<const uint4*>(xi + sb0);
    uint4* xdst = reinterpret_cast<uint4*>(sx);
    using lds_ptr = __attribute__((address_space(3))) void*;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i0 = k * kThreads + wave * 64;   // the wave's first word (uniform)
        if (i0 + lane < n16) __builtin_amdgcn_global_load_lds(xsrc + i0 + lane, (lds_ptr)(xdst + i0), 16, 0, 0);
    }
    const int s = lane >> 4, li = lane & 15;
    const Q4kSegment seg(s);
    // the sums of squares of the batch rows this lane's results belong to (RMSNorm
    // factor): loaded with the x slab, every row clamped into the batch (no branch that
    // would wait for each load on the spot), used once the slab has landed
    float4 rnp[NBT][4];
    if (rn.part) {   // uniform
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int e = 0; e < 4; ++e) rnp[bt][e] = rn.part[min(bt * 16 + 4 * s + e, batch - 1)];
    }

    const int total_rows = kDual ? 2 * rows : rows;
    const int ntile = (rows + 15) >> 4;
    constexpr int kTpu = kDual ? TPW / 2 : TPW;   // row tiles per unit
    const int nunits = (ntile + kTpu - 1) / kTpu;

    // Work split: this workgroup's balanced contiguous unit range [wa, wb) of the slab is
    // cut into (unit, superblock) items, shared out to the waves in balanced contiguous
    // ranges (so no wave carries a whole extra unit).  A unit whose items span several
    // waves belongs to the wave holding its first item; the later ones hand it their
    // partial sums through LDS after the loop.  floor(p nunits / wgs) in 32 bits:
    // p (q wgs + r) / wgs = p q + floor(p r / wgs), p r < wgs^2.
    const int uq = nunits / wgs_per_slab, ur = nunits - uq * wgs_per_slab;
    const int wa = pos * uq + pos * ur / wgs_per_slab, wb = (pos + 1) * uq + (pos + 1) * ur / wgs_per_slab;
    const int items = (wb - wa) * nsb;
    auto item0 = [&](int wv) { return wv * items / NWAVES; };
    const int ia = item0(wave), nit = item0(wave + 1) - ia;

    // tile t of unit u: row tile kTpu u + (t % kTpu) (clamped into range: a short last
    // unit repeats its last tile, whose results finish() does not write), matrix t / kTpu
    auto tile_of = [&](int u, int t) {
        const int rt = kTpu * u + (t % kTpu);
        return rt < ntile ? rt : ntile - 1;
    };
    int lu = wa + ia / nsb, lsb = ia % nsb, lit = 0;
    auto load_next = [&](Raw* dst) {
        const int64_t sb = sb0 + lsb;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const uint8_t* base = (kDual && t >= kTpu) ? w2 : w;
            F::load(base + ((int64_t)tile_of(lu, t) * nsbt + sb) * F::kBytes, lane, dst[t]);
        }
        if (lit < nit - 1) {
            ++lit;
            if (++lsb == nsb) {
                lsb = 0;
                ++lu;
            }
        }
    };
    Raw buf[DEPTH][TPW];
    if (nit > 0) {
#pragma unroll
        for (int d = 0; d < DEPTH - 1; ++d) load_next(buf[d]);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the direct loads have landed
    __syncthreads();

    // the RMSNorm factor of each batch row this lane's results belong to
    float rowf[NBT][4];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
        for (int e = 0; e < 4; ++e) rowf[bt][e] = rn.part ? row_norm_factor(rn, rnp[bt][e]) : 1.0f;

    f4_t acc[TPW][NBT];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int sbl, const Raw* r) {
        const Img& im = sx[sbl];
        f4_t C[TPW][NBT], Cm[TPW][NBT];
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) C[t][bt] = Cm[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        float dC[TPW], dM[TPW];
        h8_t bm[TPW];
        auto xload = [&](int kk, h8_t* ah, h8_t* al) {
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                ah[bt] = *reinterpret_cast<const h8_t*>(&im.x[0][bt * 16 + li][kk]);
                al[bt] = *reinterpret_cast<const h8_t*>(&im.x[1][bt * 16 + li][kk]);
            }
        };
        auto mma = [&](const h8_t* ah, const h8_t* al, const h8_t* bw) {
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt)
                    C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[bt], bw[t], C[t][bt], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt)
                    C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[bt], bw[t], C[t][bt], 0, 0, 0);
        };
        if constexpr (kQ4) {
            uint32_t slo[TPW], shi[TPW];
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
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
                h8_t bw[TPW];
#pragma unroll
                for (int t = 0; t < TPW; ++t) {
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
                mma(ah, al, bw);
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
            float scq[TPW][4];
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)r[t].d);
                dC[t] = d * 16384.0f;   // codes carry 2^-14
                dM[t] = d * 512.0f;     // -32 sc x: sums staged / 16
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
                h8_t bw[TPW];
#pragma unroll
                for (int t = 0; t < TPW; ++t) {
                    const uint4& run = (q & 1) ? r[t].b : r[t].a;
                    const uint32_t sp = h2dup(scq[t][q] * 256.0f);
                    uint32_t v[4];
#pragma unroll
                    for (int d2 = 0; d2 < 2; ++d2) {
                        const uint32_t rw = word_of(run, 2 * half + d2), hw = word_of(r[t].h, 2 * half + d2);
                        const uint32_t nb = (q >> 1) ? (rw >> 2) : (rw << 2);
                        const uint32_t code = (nb & 0x3C3C3C3Cu) | ((hw << (6 - 2 * q)) & 0xC0C0C0C0u);
                        v[2 * d2] = pk_mul_f16(code & 0x00FF00FFu, sp);
                        v[2 * d2 + 1] = pk_mul_f16((code >> 8) & 0x00FF00FFu, sp);
                    }
                    bw[t] = __builtin_bit_cast(h8_t, uint4{v[0], v[1], v[2], v[3]});
                }
                h8_t nh[NBT], nl[NBT];
                if (m < 7) xload(col(m + 1), nh, nl);
                mma(ah, al, bw);
                if (m < 7) {
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt) {
                        ah[bt] = nh[bt];
                        al[bt] = nl[bt];
                    }
                }
            }
        }
        // group-sum MFMA (the minimum term of Q4_K, the -32 offset of Q6_K)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            const h8_t am = im.g[bt * 16 + li][s];
#pragma unroll
            for (int t = 0; t < TPW; ++t)
                Cm[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bm[t], Cm[t][bt], 0, 0, 0);
        }
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float inv = im.inv[bt * 16 + 4 * s + e];
#pragma unroll
                for (int t = 0; t < TPW; ++t) {
                    float v = dC[t] * C[t][bt][e];
                    v = kQ4 ? fmaf(-dM[t], Cm[t][bt][e], v) : fmaf(dM[t], Cm[t][bt][e], v);
                    acc[t][bt][e] = fmaf(v, inv, acc[t][bt][e]);
                }
            }
    };

    // unit finished: the epilogue (one slab) or partial sums [slab][batch][virtual row]
    auto finish = [&](int u) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][bt][e] *= rowf[bt][e];
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const int rt = kTpu * u + (t % kTpu);
            const int row = 16 * rt + li;
            const bool ok = rt < ntile && row < rows;
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int b = bt * 16 + 4 * s + e;
                    const float val = acc[t][bt][e];
                    if (nslab > 1) {
                        const int v = kDual ? 2 * row + t / kTpu : row;
                        if (ok && b < batch) part[((int64_t)slab * kMaxBatchTile + b) * total_rows + v] = val;
                    } else if constexpr (kDual) {
                        if (t >= kTpu && ok && b < batch)
                            y[(int64_t)b * rows + row] = swiglu(acc[t - kTpu][bt][e], val);
                    } else if constexpr (MODE == kAccumulate) {
                        if (ok && b < batch) y[(int64_t)b * rows + row] += val;
                    } else {
                        if (ok && b < batch) y[(int64_t)b * rows + row] = val;
                    }
                }
        }
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    };

    int cu = wa + ia / nsb, csb = ia % nsb;   // (unit, superblock) being multiplied
    const int head = cu;                      // the wave's first unit ...
    const bool head_shared = csb != 0;        // ... began in an earlier wave
    f4_t hacc[TPW][NBT];                      // its partial sums, for that wave
    for (int it0 = 0; it0 < nit; it0 += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int it = it0 + d;
            load_next(buf[(d + DEPTH - 1) % DEPTH]);
            if (it < nit) {
                take_turns(wave, it);
                compute(csb, buf[d]);
                if (csb == nsb - 1) {
                    if (head_shared && cu == head) {
#pragma unroll
                        for (int t = 0; t < TPW; ++t)
#pragma unroll
                            for (int bt = 0; bt < NBT; ++bt) {
                                hacc[t][bt] = acc[t][bt];
                                acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
                            }
                    } else {
                        finish(cu);
                    }
                }
                if (++csb == nsb) {
                    csb = 0;
                    ++cu;
                }
            }
        }
    }
    // units left open: the head piece of a unit that ends inside this wave's range holds
    // only a middle part (it is the head partial), or the wave owns an unfinished unit
    const bool open = nit > 0 && csb != 0;
    const bool mid = open && head_shared && cu == head;
    if (mid) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) hacc[t][bt] = acc[t][bt];
    }
    // hand the head partials over through LDS (the x images are no longer read)
    constexpr int kSlot = TPW * NBT * 4 * 64;   // floats per wave
    static_assert(NWAVES * kSlot * sizeof(float) <= sizeof(sx), "partial slots fit in the x images");
    float* slots = reinterpret_cast<float*>(sx);
    __syncthreads();
    if (head_shared && nit > 0) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int e = 0; e < 4; ++e) slots[wave * kSlot + ((t * NBT + bt) * 4 + e) * 64 + lane] = hacc[t][bt][e];
    }
    __syncthreads();
    if (open && !mid) {   // the owner adds the pieces of the later waves in wave order
        const int end = (cu - wa + 1) * nsb;   // items of the unit end here
        for (int wv = wave + 1; wv < NWAVES && item0(wv) < end; ++wv) {
            if (item0(wv + 1) == item0(wv)) continue;   // (a wave without items holds no piece)
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[t][bt][e] += slots[wv * kSlot + ((t * NBT + bt) * 4 + e) * 64 + lane];
        }
        finish(cu);
    }
}

}  // namespace rta
