// rta_gemv.hpp -- dequant-fused matrix-vector readout for Q4_K / Q6_K on gfx950.
//
// Work decomposition (wave64):
//   A row of `cols` values is cut into slots of 64 values (S = cols/64 slots):
//     Q4_K slot = chunk j of a superblock: 32 nibble bytes, groups 2j and 2j+1
//     Q6_K slot = (half h, l0 in {0,16}) of a superblock: 16 ql bytes at
//                 64h+l0 and 64h+32+l0, 16 qh bytes at 128+32h+l0, 4 scales
//   `lpr` lanes share one row (lpr = min(64, pow2ceil(S))); a wave therefore
//   covers P = 64/lpr rows per pass and R passes per task (P*R consecutive rows).
//   Each lane streams its slot's bytes straight from HBM (16-byte loads for Q4_K,
//   4-byte loads + alignbyte for the 2-byte aligned Q6_K blocks), unpacks codes in
//   registers and accumulates code*x with v_fma_mix_f32 (the codes are binary16
//   subnormals, so the conversion is free and exact).  The per-group scale and
//   minimum are applied once per slot:  sum_i (D q_i - M) x_i = D sum q_i x_i - M sum x_i.
//   Partial sums are reduced across the row's lanes with xor shuffles.
//
// Equivalent reference: resident_math.comp:39-75 (one 32-lane subgroup per channel,
// quantizedOctet decode of resident_quant.glsl:47-94, subgroupAdd).
#pragma once
#include "rta_common.hpp"

namespace rta {

enum GemvMode { kStore = 0, kAccumulate = 1, kSwiglu = 2, kLogits = 3 };

struct GemvArgs {
    const uint8_t* w;     // matrix (gate matrix in kSwiglu)
    const uint8_t* w2;    // up matrix in kSwiglu
    int64_t row_bytes;
    int rows, cols;
    const float* x;       // [batch, cols]
    float* y;             // [batch, rows]
    float* partial;       // kLogits: [batch, ntasks] maxima per task
    int batch;            // rows of x handled by this launch (<= NB)
    int lpr;              // lanes per matrix row
    int ntasks;
};

// ---------------------------------------------------------------- Q4_K ----
struct Q4K {
    static constexpr int kBytes = 144;
    static constexpr int kRuns = 2;       // x runs per slot: [0,32) low nibbles, [32,64) high
    static constexpr int kRunLen = 32;
    struct Raw { uint4 hdr, q0, q1; };
    struct Scale { float d0, d1, m0, m1; };

    __device__ static __forceinline__ int run_col(int slot, int run) {
        return (slot >> 2) * 256 + (slot & 3) * 64 + run * 32;
    }
    __device__ static __forceinline__ void load(const uint8_t* row, int slot, Raw& r) {
        const uint8_t* blk = row + (int64_t)(slot >> 2) * kBytes;
        const int j = slot & 3;
        r.hdr = *reinterpret_cast<const uint4*>(blk);
        r.q0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * j);
        r.q1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * j);
    }
    __device__ static __forceinline__ Scale scale(const Raw& r, int slot) {
        const int j = slot & 3;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j, sc0, m0);
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j + 1, sc1, m1);
        const float d = half_lo(r.hdr.x), dmin = half_hi(r.hdr.x);
        Scale s;
        s.d0 = d * (float)sc0 * 16777216.0f;  // low-nibble codes carry 2^-24
        s.d1 = d * (float)sc1 * 1048576.0f;   // high-nibble codes carry 2^-20
        s.m0 = dmin * (float)m0;
        s.m1 = dmin * (float)m1;
        return s;
    }
    // acc[0] += sum q_lo x[0..32) * 2^-24 ; acc[1] += sum q_hi x[32..64) * 2^-20
    __device__ static __forceinline__ void dot(const Raw& r, const float* __restrict__ xs, float acc[kRuns]) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        float a0 = acc[0], a1 = acc[1], b0 = 0.0f, b1 = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t w = q[t], v = w >> 8;
            const half2_t p0 = as_codes(w & 0x000F000Fu), p1 = as_codes(v & 0x000F000Fu);
            const half2_t h0 = as_codes(w & 0x00F000F0u), h1 = as_codes(v & 0x00F000F0u);
            a0 = fmaf((float)p0.x, xs[4 * t + 0], a0);
            b0 = fmaf((float)p1.x, xs[4 * t + 1], b0);
            a0 = fmaf((float)p0.y, xs[4 * t + 2], a0);
            b0 = fmaf((float)p1.y, xs[4 * t + 3], b0);
            a1 = fmaf((float)h0.x, xs[32 + 4 * t + 0], a1);
            b1 = fmaf((float)h1.x, xs[32 + 4 * t + 1], b1);
            a1 = fmaf((float)h0.y, xs[32 + 4 * t + 2], a1);
            b1 = fmaf((float)h1.y, xs[32 + 4 * t + 3], b1);
        }
        acc[0] = a0 + b0;
        acc[1] = a1 + b1;
    }
    __device__ static __forceinline__ float combine(const Scale& s, const float acc[kRuns], const float X[kRuns]) {
        float v = s.d0 * acc[0];
        v = fmaf(-s.m0, X[0], v);
        v = fmaf(s.d1, acc[1], v);
        v = fmaf(-s.m1, X[1], v);
        return v;
    }
};

// ---------------------------------------------------------------- Q6_K ----
struct Q6K {
    static constexpr int kBytes = 210;
    static constexpr int kRuns = 4;       // run k: values l0 + [0,16) + 32k of half h
    static constexpr int kRunLen = 16;
    struct Raw { uint32_t a[4], b[4], h[4]; uint32_t s; uint32_t d; };
    struct Scale { float d[4]; };

    __device__ static __forceinline__ int run_col(int slot, int run) {
        const int hh = (slot >> 1) & 1, l0 = (slot & 1) * 16;
        return (slot >> 2) * 256 + hh * 128 + l0 + 32 * run;
    }
    // Loads 16 bytes that start at a 2-byte aligned address p (never beyond p + 20).
    __device__ static __forceinline__ void load16(const uint8_t* p, uint32_t out[4]) {
        const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
        const uint32_t mis = (uint32_t)(addr & 3u);
        const uint32_t* a = reinterpret_cast<const uint32_t*>(addr - mis);
        uint32_t w[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) w[i] = a[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = funnel(w[i], w[i + 1], mis);
    }
    __device__ static __forceinline__ void load(const uint8_t* row, int slot, Raw& r) {
        const uint8_t* blk = row + (int64_t)(slot >> 2) * kBytes;
        const int hh = (slot >> 1) & 1, l0 = (slot & 1) * 16;
        load16(blk + 64 * hh + l0, r.a);
        load16(blk + 64 * hh + 32 + l0, r.b);
        load16(blk + 128 + 32 * hh + l0, r.h);
        // scale bytes 192 + 8h + l0/16 + {0,2,4,6}: four 2-byte aligned halfwords
        const uint16_t* sp = reinterpret_cast<const uint16_t*>(blk + 192 + 8 * hh);
        const uint32_t pick = (uint32_t)(l0 >> 4) * 8u;
        uint32_t s = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) s |= (((uint32_t)sp[k] >> pick) & 255u) << (8 * k);
        r.s = s;
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
    __device__ static __forceinline__ Scale scale(const Raw& r, int) {
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)r.d);
        Scale s;
#pragma unroll
        for (int k = 0; k < 4; ++k) s.d[k] = d * (float)(int8_t)((r.s >> (8 * k)) & 255u);
        return s;
    }
    __device__ static __forceinline__ void dot(const Raw& r, const float* __restrict__ xs, float acc[kRuns]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t a = r.a[t], b = r.b[t], h = r.h[t];
            uint32_t c[4];
            c[0] = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
            c[1] = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
            c[2] = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
            c[3] = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const half2_t p = as_codes(c[k] & 0x00FF00FFu), q = as_codes((c[k] >> 8) & 0x00FF00FFu);
                const float* xr = xs + 16 * k + 4 * t;
                float v = acc[k];
                v = fmaf((float)p.x, xr[0], v);
                v = fmaf((float)q.x, xr[1], v);
                v = fmaf((float)p.y, xr[2], v);
                v = fmaf((float)q.y, xr[3], v);
                acc[k] = v;
            }
        }
    }
    __device__ static __forceinline__ float combine(const Scale& s, const float acc[kRuns], const float X[kRuns]) {
        // sum (c-32) x = sum c x - 32 sum x ; codes carry 2^-24
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) v = fmaf(s.d[k], fmaf(acc[k], 16777216.0f, -32.0f * X[k]), v);
        return v;
    }
};

template <int FMT> struct FmtOf;
template <> struct FmtOf<RTA_Q4_K> { using T = Q4K; };
template <> struct FmtOf<RTA_Q6_K> { using T = Q6K; };

// Loads the 64 x values of one slot for batch row b, and the per-run sums.
template <class F>
__device__ __forceinline__ void load_x(const float* __restrict__ x, int cols, int b, int slot,
                                       float xs[64], float X[F::kRuns]) {
    const float* xb = x + (int64_t)b * cols;
#pragma unroll
    for (int run = 0; run < F::kRuns; ++run) {
        const float4* p = reinterpret_cast<const float4*>(xb + F::run_col(slot, run));
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < F::kRunLen / 4; ++i) {
            const float4 v = p[i];
            xs[run * F::kRunLen + 4 * i + 0] = v.x;
            xs[run * F::kRunLen + 4 * i + 1] = v.y;
            xs[run * F::kRunLen + 4 * i + 2] = v.z;
            xs[run * F::kRunLen + 4 * i + 3] = v.w;
            s += (v.x + v.y) + (v.z + v.w);
        }
        X[run] = s;
    }
}

// NB: batch rows per launch (x rows), R: row passes per task.
template <int FMT, int NB, int R, int MODE>
__global__ void __launch_bounds__(256) gemv_kquant_kernel(const GemvArgs a) {
    using F = typename FmtOf<FMT>::T;
    constexpr bool kDual = MODE == kSwiglu;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int S = a.cols >> 6;
    const int lpr = a.lpr, P = kWave / lpr;
    const int sub = lane / lpr, lir = lane - sub * lpr;
    const int ks = (S + lpr - 1) / lpr;
    const int rows_per_task = P * R;

    for (int task = blockIdx.x * 4 + wave; task < a.ntasks; task += gridDim.x * 4) {
        const int row0 = task * rows_per_task + sub;
        float acc[R][NB], acc2[R][NB];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[r][b] = acc2[r][b] = 0.0f;

        for (int k = 0; k < ks; ++k) {
            const int slot = lir + k * lpr;
            if (slot < S) {
                typename F::Raw raw[R], raw2[kDual ? R : 1];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int row = min(row0 + P * r, a.rows - 1);   // clamped rows are discarded
                    F::load(a.w + (int64_t)row * a.row_bytes, slot, raw[r]);
                    if constexpr (kDual) F::load(a.w2 + (int64_t)row * a.row_bytes, slot, raw2[r]);
                }
                typename F::Scale sc[R], sc2[kDual ? R : 1];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    sc[r] = F::scale(raw[r], slot);
                    if constexpr (kDual) sc2[r] = F::scale(raw2[r], slot);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    if (b < a.batch) {
                        float xs[64], X[F::kRuns];
                        load_x<F>(a.x, a.cols, b, slot, xs, X);
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            float part[F::kRuns];
#pragma unroll
                            for (int i = 0; i < F::kRuns; ++i) part[i] = 0.0f;
                            F::dot(raw[r], xs, part);
                            acc[r][b] += F::combine(sc[r], part, X);
                            if constexpr (kDual) {
#pragma unroll
                                for (int i = 0; i < F::kRuns; ++i) part[i] = 0.0f;
                                F::dot(raw2[r], xs, part);
                                acc2[r][b] += F::combine(sc2[r], part, X);
                            }
                        }
                    }
                }
            }
        }
        // Reduce across the lpr lanes of each row; every lane of the row gets the sum.
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[r][b] = group_sum(acc[r][b], lpr);
                if constexpr (kDual) acc2[r][b] = group_sum(acc2[r][b], lpr);
            }

        float local_max[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) local_max[b] = -INFINITY;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + P * r;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= a.batch || row >= a.rows) continue;
                float* out = a.y + (int64_t)b * a.rows + row;
                const float v = acc[r][b];
                if constexpr (MODE == kLogits) local_max[b] = fmaxf(local_max[b], v);
                if (lir == 0) {
                    if constexpr (MODE == kStore || MODE == kLogits) *out = v;
                    else if constexpr (MODE == kAccumulate) *out += v;
                    else *out = swiglu(v, acc2[r][b]);
                }
            }
        }
        if constexpr (MODE == kLogits) {
            // max over the P rows of this pass set: lanes sub*lpr hold row partials
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float m = local_max[b];
                for (int off = lpr; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
                if (lane == 0 && b < a.batch) a.partial[(int64_t)b * a.ntasks + task] = m;
            }
        }
    }
}

// ------------------------------------------------------- F32 / F16 / BF16 ----
// One wave per row: plain element formats (resident_quant.glsl:7-9).
template <int FMT>
__device__ __forceinline__ float plain_value(const uint8_t* row, int c) {
    if constexpr (FMT == RTA_F32) return reinterpret_cast<const float*>(row)[c];
    else if constexpr (FMT == RTA_F16) return (float)reinterpret_cast<const _Float16*>(row)[c];
    else return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(row)[c] << 16);
}

template <int FMT, int MODE>
__global__ void __launch_bounds__(256) gemv_plain_kernel(const GemvArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ntasks = a.rows;  // one row per task
    for (int row = blockIdx.x * 4 + wave; row < ntasks; row += gridDim.x * 4) {
        const uint8_t* wr = a.w + (int64_t)row * a.row_bytes;
        const uint8_t* wr2 = MODE == kSwiglu ? a.w2 + (int64_t)row * a.row_bytes : nullptr;
        for (int b = 0; b < a.batch; ++b) {
            const float* xb = a.x + (int64_t)b * a.cols;
            float s = 0.0f, s2 = 0.0f;
            for (int c = lane; c < a.cols; c += kWave) {
                s = fmaf(plain_value<FMT>(wr, c), xb[c], s);
                if constexpr (MODE == kSwiglu) s2 = fmaf(plain_value<FMT>(wr2, c), xb[c], s2);
            }
            s = group_sum(s, kWave);
            if constexpr (MODE == kSwiglu) s2 = group_sum(s2, kWave);
            if (lane == 0) {
                float* out = a.y + (int64_t)b * a.rows + row;
                if constexpr (MODE == kStore || MODE == kLogits) *out = s;
                else if constexpr (MODE == kAccumulate) *out += s;
                else *out = swiglu(s, s2);
                if constexpr (MODE == kLogits) a.partial[(int64_t)b * a.ntasks + row] = s;
            }
        }
    }
}

}  // namespace rta
