// rta_gemm.hpp -- batched (>= 8 rows) dequant-fused readout on the gfx950 matrix cores.
//
// y[b, r] = sum_k W[r, k] x[b, k] for a batch of up to 32 x rows per launch, with
// v_mfma_f32_16x16x32_f16 (fp32 accumulation):
//   A operand  x, prepared once per call (xprep_kernel): per batch row a power-of-two
//              scale s_b puts max|x_b s_b| in [2^13, 2^14); x s_b is split into
//              binary16 hi + lo (22 significant bits), both multiplied in.
//   B operand  the weights, built in registers as exact binary16 integers:
//                Q4_K  sc_g * q          (<= 945)   = fma(1024 + q, sc, -1024 sc)
//                Q6_K  sc * (q - 32)     = ((1024 + q) - 1056) * sc, exact for
//                                         |product| <= 2048; beyond that (|sc| > 64)
//                                         it rounds to 11 bits, < 2^-12 relative
//              with packed binary16 ops on two codes at a time (1024 + q is the code
//              OR 0x6400, an exact binary16 integer).
//              So a superblock accumulates across all its groups and d (and the
//              Q4_K minimum term dmin * sum_g m_g X_g, one more MFMA over the group
//              sums) is applied once per superblock and output.
//   Layout     lane l of a wave: weight row l%16 / k segment 8*(l/16) (B operand),
//              batch row l%16 / k segment 8*(l/16) (A operand), and it owns outputs
//              (batch 4*(l/16)+e, row l%16) -- the row whose header it loaded.
// A workgroup (4 waves) covers 64*RT rows x one K slab; x for the slab is staged
// superblock by superblock in double-buffered LDS and shared by the 4 waves; the
// weights of the next superblock are prefetched into registers.  K slabs > 1 write
// partial sums that gemm_reduce_kernel adds in a fixed order (deterministic).
//
// Equivalent reference: the batched projection pipelines (optical_resident.cpp:168,343,
// matrixRows 4/8/16) and resident_batch2.comp (which accumulates in fp16; not copied).
#pragma once
#include "rta_gemv.hpp"

namespace rta {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2v_t __attribute__((ext_vector_type(2)));

constexpr int kMaxBatchTile = 32;  // batch rows per GEMM launch
constexpr int kXpad = 8;           // f16 padding per staged x row (bank spread)

struct GemmX {           // prepared x (workspace), batch padded to 32
    _Float16* hi;        // [32][cols]
    _Float16* lo;        // [32][cols]
    _Float16* gs;        // [32][cols/32][2] group sums / 32, hi and lo
    float* inv;          // [32] 1/s_b
};

// ---------------------------------------------------------------- x prep ----
__global__ void __launch_bounds__(256) xprep_kernel(const float* __restrict__ x, int cols, int batch, GemmX p) {
    __shared__ float red[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* xb = x + (int64_t)b * cols;
    _Float16* hi = p.hi + (int64_t)b * cols;
    _Float16* lo = p.lo + (int64_t)b * cols;
    _Float16* gs = p.gs + (int64_t)b * (cols / 32) * 2;
    if (b >= batch) {   // padding rows of the 32-row tile: zeros
        for (int c = tid; c < cols; c += 256) hi[c] = lo[c] = (_Float16)0.0f;
        for (int g = tid; g < cols / 32; g += 256) gs[2 * g] = gs[2 * g + 1] = (_Float16)0.0f;
        if (tid == 0) p.inv[b] = 0.0f;
        return;
    }
    float m = 0.0f;
    for (int c = tid; c < cols; c += 256) m = fmaxf(m, fabsf(xb[c]));
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (m > 0.0f && isfinite(m)) (void)frexpf(m, &e);
    const float s = ldexpf(1.0f, 14 - e);          // m * s in [2^13, 2^14)
    if (tid == 0) p.inv[b] = ldexpf(1.0f, e - 14);
    for (int c = tid; c < cols; c += 256) {
        const float v = xb[c] * s;
        const _Float16 h = (_Float16)v;
        hi[c] = h;
        lo[c] = (_Float16)(v - (float)h);
    }
    for (int g = tid; g < cols / 32; g += 256) {
        float acc = 0.0f;
        for (int i = 0; i < 32; ++i) acc += xb[32 * g + i] * s;
        const float v = acc * (1.0f / 32.0f);      // |v| < 2^14: fits binary16
        const _Float16 h = (_Float16)v;
        gs[2 * g] = h;
        gs[2 * g + 1] = (_Float16)(v - (float)h);
    }
}

__device__ __forceinline__ uint32_t pk_fma_f16(uint32_t a, uint32_t b, uint32_t c) {
    const h2v_t r = __builtin_bit_cast(h2v_t, a) * __builtin_bit_cast(h2v_t, b) + __builtin_bit_cast(h2v_t, c);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t pk_add_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v_t, a) + __builtin_bit_cast(h2v_t, b));
}
__device__ __forceinline__ uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v_t, a) * __builtin_bit_cast(h2v_t, b));
}
constexpr uint32_t kMinus1056 = 0xE420E420u;   // (-1056.0, -1056.0) in binary16

// (f16(v), f16(v)) for a small exact integer v
__device__ __forceinline__ uint32_t h2dup(float v) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}

// -------------------------------------------------------- weight operand ----
// Per lane: row l%16 of one 16-row tile, k segment s = l/16 of every 32-value chunk.
struct Q4KMma {
    static constexpr int kBytes = 144;
    struct Raw { uint4 hdr; uint2 q[4]; };   // q[j] = bytes 16+32j+8s .. +8
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ blk, int s, Raw& r) {
        r.hdr = *reinterpret_cast<const uint4*>(blk);
#pragma unroll
        for (int j = 0; j < 4; ++j) r.q[j] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * j + 8 * s);
    }
};

struct Q6KMma {
    static constexpr int kBytes = 210;
    // half h: ql runs at 64h + 8s and 64h + 32 + 8s, qh run at 128 + 32h + 8s (8 bytes
    // each), loaded as 3 dwords from the 4-byte aligned address below; scales 192..207; d.
    struct Raw { uint32_t a[2][3], b[2][3], h[2][3]; uint32_t sc[5]; uint32_t d; uint32_t mis; };
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ blk, int s, Raw& r) {
        const uintptr_t addr = reinterpret_cast<uintptr_t>(blk);
        const uint32_t mis = (uint32_t)(addr & 3u);
        const uint32_t* a = reinterpret_cast<const uint32_t*>(addr - mis);
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

// Spreads bytes i, i+1 of w into the low bytes of the two halves.
__device__ __forceinline__ uint32_t spread(uint32_t w, int i) {
    return __builtin_amdgcn_perm(w, w, i == 0 ? 0x0C010C00u : 0x0C030C02u);
}

template <int FMT, int RT, int NBT, int XS, int MODE>
__global__ void __launch_bounds__(256) gemm_mfma_kernel(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, const int64_t row_bytes, const int rows,
    const int cols, const GemmX xp, const int batch, float* __restrict__ y, float* __restrict__ part,
    const int row_blocks, const int sb_per_slab) {
    constexpr bool kQ4 = FMT == RTA_Q4_K;
    constexpr int kStride = 256 + kXpad;                       // staged x row, f16 elements
    __shared__ _Float16 s_xh[2][kMaxBatchTile][kStride];
    __shared__ _Float16 s_xl[XS == 2 ? 2 : 1][XS == 2 ? kMaxBatchTile : 1][XS == 2 ? kStride : 1];
    __shared__ _Float16 s_gs[2][kMaxBatchTile][16];            // 8 groups x (hi, lo) per batch row

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rb = blockIdx.x % row_blocks, slab = blockIdx.x / row_blocks;
    const int sb0 = slab * sb_per_slab;
    const int nsb = min(sb_per_slab, cols / 256 - sb0);
    const int s = lane >> 4, li = lane & 15;
    const int total_rows = MODE == kSwiglu ? 2 * rows : rows;

    // rows of this lane's RT tiles (clamped: out-of-range rows are computed and dropped)
    const uint8_t* rowp[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        int r = rb * 64 * RT + wave * 16 * RT + t * 16 + li;
        r = min(r, total_rows - 1);
        const uint8_t* base = (MODE == kSwiglu && r >= rows) ? w2 + (int64_t)(r - rows) * row_bytes
                                                             : w + (int64_t)r * row_bytes;
        rowp[t] = base;
    }

    auto stage = [&](int sb, int buf) {   // x of superblock sb -> LDS buffer
        const int k0 = sb * 256;
        // 32 rows x 256 f16 = 32 x 32 chunks of 16 bytes per array
        for (int i = tid; i < kMaxBatchTile * 32; i += 256) {
            const int b = i >> 5, c = (i & 31) * 8;
            *reinterpret_cast<uint4*>(&s_xh[buf][b][c]) = *reinterpret_cast<const uint4*>(xp.hi + (int64_t)b * cols + k0 + c);
            if constexpr (XS == 2)
                *reinterpret_cast<uint4*>(&s_xl[buf][b][c]) = *reinterpret_cast<const uint4*>(xp.lo + (int64_t)b * cols + k0 + c);
        }
        if constexpr (kQ4) {
            if (tid < kMaxBatchTile * 4) {   // 8 groups x 2 f16 = 32 bytes per batch row
                const int b = tid >> 2, q = tid & 3;
                *reinterpret_cast<uint2*>(&s_gs[buf][b][4 * q]) =
                    *reinterpret_cast<const uint2*>(xp.gs + ((int64_t)b * (cols / 32) + sb * 8) * 2 + 4 * q);
            }
        }
    };

    using Raw = typename std::conditional<kQ4, Q4KMma, Q6KMma>::type::Raw;
    Raw cur[RT], nxt[RT];
    auto load_w = [&](int sb, Raw* dst) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            if constexpr (kQ4) Q4KMma::load(rowp[t] + (int64_t)sb * 144, s, dst[t]);
            else Q6KMma::load(rowp[t] + (int64_t)sb * 210, s, dst[t]);
        }
    };

    f4_t acc[RT][NBT];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) acc[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

    if (nsb > 0) {
        stage(sb0, 0);
        load_w(sb0, cur);
    }
    __syncthreads();
    for (int i = 0; i < nsb; ++i) {
        const int buf = i & 1;
        if (i + 1 < nsb) {
            stage(sb0 + i + 1, buf ^ 1);
            load_w(sb0 + i + 1, nxt);
        }
        f4_t C[RT][NBT], Cm[RT][NBT];
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) C[t][bt] = Cm[t][bt] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        float dsc[RT], dmn[RT];

        if constexpr (kQ4) {
            uint32_t scp[RT][8], mcp[RT][8];   // (sc, sc) and (-1024 sc, -1024 sc) per group
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const uint4 h = cur[t].hdr;
                dsc[t] = half_lo(h.x);
                dmn[t] = half_hi(h.x) * 32.0f;        // group sums are staged / 32
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    uint32_t sc, m;
                    q4k_scale_min(h.y, h.z, h.w, g, sc, m);
                    scp[t][g] = h2dup((float)sc);
                    mcp[t][g] = h2dup(-1024.0f * (float)sc);
                    (void)m;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                h8_t bw[RT][2];   // weight operand for groups 2j (low nibbles), 2j+1 (high)
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    const uint32_t w0 = cur[t].q[j].x, w1 = cur[t].q[j].y;
                    const uint32_t tt[4] = {spread(w0, 0), spread(w0, 2), spread(w1, 0), spread(w1, 2)};
                    uint32_t lo[4], hi[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t pl = (tt[e] & 0x000F000Fu) | 0x64006400u;
                        const uint32_t ph = ((tt[e] >> 4) & 0x000F000Fu) | 0x64006400u;
                        lo[e] = pk_fma_f16(pl, scp[t][2 * j], mcp[t][2 * j]);
                        hi[e] = pk_fma_f16(ph, scp[t][2 * j + 1], mcp[t][2 * j + 1]);
                    }
                    bw[t][0] = __builtin_bit_cast(h8_t, uint4{lo[0], lo[1], lo[2], lo[3]});
                    bw[t][1] = __builtin_bit_cast(h8_t, uint4{hi[0], hi[1], hi[2], hi[3]});
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int kk = (2 * j + half) * 32 + 8 * s;       // k offset inside the superblock
#pragma unroll
                    for (int bt = 0; bt < NBT; ++bt) {
                        const h8_t ah = *reinterpret_cast<const h8_t*>(&s_xh[buf][bt * 16 + li][kk]);
#pragma unroll
                        for (int t = 0; t < RT; ++t)
                            C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw[t][half], C[t][bt], 0, 0, 0);
                        if constexpr (XS == 2) {
                            const h8_t al = *reinterpret_cast<const h8_t*>(&s_xl[buf][bt * 16 + li][kk]);
#pragma unroll
                            for (int t = 0; t < RT; ++t)
                                C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw[t][half], C[t][bt], 0, 0, 0);
                        }
                    }
                }
            }
            // minimum term: sum_g m_g (X_g hi + X_g lo); k 0..7 hi, 8..15 lo, 16..31 zero
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                h8_t bm;
                const uint4 h = cur[t].hdr;
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    uint32_t sc, m;
                    q4k_scale_min(h.y, h.z, h.w, g, sc, m);
                    bm[g] = s < 2 ? (_Float16)(float)m : (_Float16)0.0f;
                    (void)sc;
                }
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt) {
                    h8_t am;
                    const _Float16* gsrow = &s_gs[buf][bt * 16 + li][0];
#pragma unroll
                    for (int g = 0; g < 8; ++g) am[g] = s < 2 ? gsrow[2 * g + s] : (_Float16)0.0f;
                    Cm[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bm, Cm[t][bt], 0, 0, 0);
                }
            }
        } else {
            // Q6_K: chunk c (32 values) = half c/4, l = 32(c%4) + 8s + [0,8); group 16 = 2c + s/2
#pragma unroll
            for (int t = 0; t < RT; ++t) dsc[t] = (float)__builtin_bit_cast(_Float16, (uint16_t)cur[t].d);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int hh = c >> 2, q4 = c & 3;
                h8_t bw[RT];
#pragma unroll
                for (int t = 0; t < RT; ++t) {
                    const Raw& r = cur[t];
                    const uint32_t* run = (q4 & 1) ? r.b[hh] : r.a[hh];
                    const uint32_t a0 = funnel(run[0], run[1], r.mis), a1 = funnel(run[1], run[2], r.mis);
                    const uint32_t h0 = funnel(r.h[hh][0], r.h[hh][1], r.mis), h1 = funnel(r.h[hh][1], r.h[hh][2], r.mis);
                    const int nib = (q4 >> 1) * 4, hs = 2 * q4;
                    const uint32_t c0 = ((a0 >> nib) & 0x0F0F0F0Fu) | (((h0 >> hs) & 0x03030303u) << 4);
                    const uint32_t c1 = ((a1 >> nib) & 0x0F0F0F0Fu) | (((h1 >> hs) & 0x03030303u) << 4);
                    const int gidx = 8 * hh + 2 * q4 + (s >> 1);      // scale index 0..15
                    const uint32_t sw = funnel(r.sc[gidx >> 2], r.sc[(gidx >> 2) + 1], r.mis);
                    const float scf = (float)(int8_t)((sw >> (8 * (gidx & 3))) & 255u);
                    const uint32_t sp = h2dup(scf);
                    const uint32_t tt[4] = {spread(c0, 0), spread(c0, 2), spread(c1, 0), spread(c1, 2)};
                    uint32_t v[4];
                    // (1024 + c) - 1056 = c - 32 exactly, then times the int8 scale
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = pk_mul_f16(pk_add_f16(tt[e] | 0x64006400u, kMinus1056), sp);
                    bw[t] = __builtin_bit_cast(h8_t, uint4{v[0], v[1], v[2], v[3]});
                }
                const int kk = c * 32 + 8 * s;
#pragma unroll
                for (int bt = 0; bt < NBT; ++bt) {
                    const h8_t ah = *reinterpret_cast<const h8_t*>(&s_xh[buf][bt * 16 + li][kk]);
#pragma unroll
                    for (int t = 0; t < RT; ++t)
                        C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bw[t], C[t][bt], 0, 0, 0);
                    if constexpr (XS == 2) {
                        const h8_t al = *reinterpret_cast<const h8_t*>(&s_xl[buf][bt * 16 + li][kk]);
#pragma unroll
                        for (int t = 0; t < RT; ++t)
                            C[t][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bw[t], C[t][bt], 0, 0, 0);
                    }
                }
            }
        }
        // superblock scale: acc += d C - dmin 32 Cmin  (per lane: its own row)
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = fmaf(dsc[t], C[t][bt][e], acc[t][bt][e]);
                    if constexpr (kQ4) v = fmaf(-dmn[t], Cm[t][bt][e], v);
                    acc[t][bt][e] = v;
                }
        if (i + 1 < nsb) {
#pragma unroll
            for (int t = 0; t < RT; ++t) cur[t] = nxt[t];
        }
        __syncthreads();
    }

    // outputs: batch 16 bt + 4 s + e, row (tile base) + li
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int r = rb * 64 * RT + wave * 16 * RT + t * 16 + li;
        if (r >= total_rows) continue;
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int b = bt * 16 + 4 * s + e;
                if (b >= batch) continue;
                const float v = acc[t][bt][e] * xp.inv[b];
                part[((int64_t)slab * kMaxBatchTile + b) * total_rows + r] = v;
            }
    }
}

// Adds the K-slab partials in slab order and applies the epilogue.
// kLogits also writes per-block maxima (partial[b * gridDim.x + block]) for the argmax.
template <int MODE>
__global__ void __launch_bounds__(256) gemm_reduce_kernel(const float* __restrict__ part, int nslab, int rows,
                                                          int batch, float* __restrict__ y, float* __restrict__ pmax) {
    const int total_rows = MODE == kSwiglu ? 2 * rows : rows;
    const int b = blockIdx.y;
    const int r = blockIdx.x * 256 + threadIdx.x;
    float v = -INFINITY;
    if (r < rows && b < batch) {
        float s = 0.0f, s2 = 0.0f;
        for (int k = 0; k < nslab; ++k) {
            const float* p = part + ((int64_t)k * kMaxBatchTile + b) * total_rows;
            s += p[r];
            if constexpr (MODE == kSwiglu) s2 += p[rows + r];
        }
        float* out = y + (int64_t)b * rows + r;
        if constexpr (MODE == kStore || MODE == kLogits) *out = s;
        else if constexpr (MODE == kAccumulate) *out += s;
        else *out = swiglu(s, s2);
        v = s;
    }
    if constexpr (MODE == kLogits) {
        for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
        __shared__ float red[4];
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
        __syncthreads();
        if (threadIdx.x == 0 && b < batch)
            pmax[(int64_t)b * gridDim.x + blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
}

}  // namespace rta
