// rta_gemv.hpp -- dequant-fused matrix-vector readout for Q4_K / Q6_K on gfx950.
//
// Work decomposition (wave64):
//   A row of `cols` values is cut into slots of 64 values (S = cols/64 slots):
//     Q4_K slot = chunk j of a superblock: 32 nibble bytes, groups 2j and 2j+1
//     Q6_K slot = (half h, l0 in {0,16}) of a superblock: 16 ql bytes at
//                 64h+l0 and 64h+32+l0, 16 qh bytes at 128+32h+l0, 4 scales
//   Each lane owns one slot position for the whole kernel, so its 64 x values
//   and their per-run sums stay in registers while the lane streams that slot
//   of row after row.  A row is covered by `lpr` lanes of one wave when
//   S <= 64 (P = 64/lpr rows per pass), or by KW = S/64 waves of one
//   workgroup when S > 64 (partials combined through LDS).
//   Weights stream straight from HBM (16-byte loads for Q4_K; 4-byte loads plus
//   alignbyte for the 2-byte aligned Q6_K blocks) one task ahead of the
//   arithmetic (ping-pong register buffers).  Codes are unpacked in registers
//   into binary16 subnormals c * 2^-24, so v_fma_mix_f32 converts and
//   accumulates in one instruction; the group scale and minimum are applied once
//   per slot:  sum_i (D q_i - M) x_i = D sum q_i x_i - M sum x_i.
//
// Equivalent reference: resident_math.comp:39-75 (one 32-lane subgroup per channel,
// quantizedOctet decode of resident_quant.glsl:47-94, subgroupAdd).
#pragma once
#include "rta_common.hpp"

namespace rta {

enum GemvMode { kStore = 0, kAccumulate = 1, kSwiglu = 2, kLogits = 3 };

// ------------------------------------------------------------ reductions ----
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of `width` lanes (power of two, 4..64); every lane of
// a group ends with the group sum.  quad_perm xor1/xor2, half-row and row
// mirrors (DPP), then xor 16 / 32 by the row swaps (v_permlane16/32_swap).
// SWAPS false: xor 16 / 32 through ds_bpermute instead (the same sums; fewer registers
// in the three-wave blocks, which the row swaps push past three waves per SIMD).
template <bool SWAPS = true>
__device__ __forceinline__ float lane_group_sum(float v, int width) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    if (width == 4) return v;
    v += dpp<0x141>(v);  // row_half_mirror
    if (width == 8) return v;
    v += dpp<0x140>(v);  // row_mirror
    if (width == 16) return v;
    v = SWAPS ? add_xor16(v) : v + __shfl_xor(v, 16, kWave);
    if (width == 32) return v;
    return SWAPS ? add_xor32(v) : v + __shfl_xor(v, 32, kWave);
}

// Max over the lanes that share lane % lpr (lpr a power of two <= 64): every lane ends
// with the maximum of its class (exact in any order).  quad_perm xor1 / xor2, row_ror 4
// and 8 (DPP; a class inside a row is closed under those rotations), then the row swaps.
__device__ __forceinline__ float max_across_groups(float v, int lpr) {
    if (lpr <= 1) v = fmaxf(v, dpp<0xB1>(v));
    if (lpr <= 2) v = fmaxf(v, dpp<0x4E>(v));
    if (lpr <= 4) v = fmaxf(v, dpp<0x124>(v));   // row_ror:4
    if (lpr <= 8) v = fmaxf(v, dpp<0x128>(v));   // row_ror:8
    if (lpr <= 16) v = max_xor16(v);
    if (lpr <= 32) v = max_xor32(v);
    return v;
}

// ---------------------------------------------------------------- Q4_K ----
struct Q4K {
    static constexpr int kBytes = 144;
    static constexpr int kRuns = 2;  // x runs per slot: [0,32) low nibbles, [32,64) high
    static constexpr int kRunLen = 32;
    struct Raw { uint4 hdr, q0, q1; };

    __device__ static __forceinline__ int run_col(int slot, int run) {
        return (slot >> 2) * 256 + (slot & 3) * 64 + run * 32;
    }
    // Inverse of run_col: slot * 64 + position of column col inside its slot's x values.
    __device__ static __forceinline__ int place(int col) { return col; }
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ row, int slot, Raw& r) {
        const uint8_t* blk = row + (slot >> 2) * kBytes;
        const int j = slot & 3;
        r.hdr = *reinterpret_cast<const uint4*>(blk);
        r.q0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * j);
        r.q1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * j);
    }
    // Contribution of one slot: D0 sum q_lo x - M0 X0 + D1 sum q_hi x - M1 X1.
    __device__ static __forceinline__ float slot_dot(const Raw& r, int slot, const float* xs, const float* X) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
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
        const int j = slot & 3;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j, sc0, m0);
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j + 1, sc1, m1);
        const float d = half_lo(r.hdr.x), dmin = half_hi(r.hdr.x);
        // low-nibble codes carry 2^-24, high-nibble codes 2^-20
        float v = (d * 16777216.0f) * (float)sc0 * (a0 + b0);
        v = fmaf(-(dmin * (float)m0), X[0], v);
        v = fmaf((d * 1048576.0f) * (float)sc1, a1 + b1, v);
        return fmaf(-(dmin * (float)m1), X[1], v);
    }
};

// ---------------------------------------------------------------- Q6_K ----
struct Q6K {
    static constexpr int kBytes = 210;
    static constexpr int kRuns = 4;  // run k: values l0 + [0,16) + 32k of half h
    static constexpr int kRunLen = 16;
    // Raw dwords from the 4-byte aligned address below each run; funnelled later.
    struct Raw { uint32_t a[5], b[5], h[5], s[3], d, mis; };

    __device__ static __forceinline__ int run_col(int slot, int run) {
        const int hh = (slot >> 1) & 1, l0 = (slot & 1) * 16;
        return (slot >> 2) * 256 + hh * 128 + l0 + 32 * run;
    }
    __device__ static __forceinline__ int place(int col) {
        const int cc = col & 255, hh = cc >> 7, run = (cc & 127) >> 5, l = cc & 31;
        return ((col >> 8) * 4 + hh * 2 + (l >> 4)) * 64 + run * 16 + (l & 15);
    }
    // Every read lies inside the 210-byte block (the last dword of each run and
    // the third scale dword are only consumed when the block is 2-byte aligned).
    __device__ static __forceinline__ void load(const uint8_t* __restrict__ row, int slot, Raw& r) {
        const uint8_t* blk = row + (slot >> 2) * kBytes;
        const int hh = (slot >> 1) & 1, l0 = (slot & 1) * 16;
        // aligned down by pointer arithmetic, which keeps the global address space
        const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const uint32_t* a = reinterpret_cast<const uint32_t*>(blk - mis);
        const int ia = (64 * hh + l0) >> 2, ib = (64 * hh + 32 + l0) >> 2, ih = (128 + 32 * hh + l0) >> 2;
        const int is = (192 + 8 * hh) >> 2;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            r.a[i] = a[ia + i];
            r.b[i] = a[ib + i];
            r.h[i] = a[ih + i];
        }
        r.s[0] = a[is];
        r.s[1] = a[is + 1];
        r.s[2] = a[is + 1 + (mis ? 1 : 0)];
        r.d = *reinterpret_cast<const uint16_t*>(blk + 208);
        r.mis = mis;
    }
    __device__ static __forceinline__ float slot_dot(const Raw& r, int slot, const float* xs, const float* X) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t a = funnel(r.a[t], r.a[t + 1], r.mis);
            const uint32_t b = funnel(r.b[t], r.b[t + 1], r.mis);
            const uint32_t h = funnel(r.h[t], r.h[t + 1], r.mis);
            const uint32_t ha = h & 0x33333333u, hb = (h >> 2) & 0x33333333u;
            uint32_t c[4];
            c[0] = (a & 0x0F0F0F0Fu) | ((ha << 4) & 0xF0F0F0F0u);
            c[1] = (b & 0x0F0F0F0Fu) | ((hb << 4) & 0xF0F0F0F0u);
            c[2] = ((a >> 4) & 0x0F0F0F0Fu) | (ha & 0xF0F0F0F0u);
            c[3] = ((b >> 4) & 0x0F0F0F0Fu) | (hb & 0xF0F0F0F0u);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const half2_t p = as_codes(c[k] & 0x00FF00FFu);
                const half2_t q = as_codes(__builtin_amdgcn_perm(c[k], c[k], 0x0C030C01u));
                const float* xr = xs + 16 * k + 4 * t;
                float v = acc[k];
                v = fmaf((float)p.x, xr[0], v);
                v = fmaf((float)q.x, xr[1], v);
                v = fmaf((float)p.y, xr[2], v);
                v = fmaf((float)q.y, xr[3], v);
                acc[k] = v;
            }
        }
        // scales 8h + l0/16 + {0,2,4,6}: bytes (l0/16) + 2k of the half's 8 scale bytes
        const uint32_t s_lo = funnel(r.s[0], r.s[1], r.mis), s_hi = funnel(r.s[1], r.s[2], r.mis);
        const uint32_t pick = (uint32_t)(slot & 1) * 8u;
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)r.d);
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t word = k < 2 ? s_lo : s_hi;
            const int sc = (int)(int8_t)((word >> (16 * (k & 1) + pick)) & 255u);
            // sum (c-32) x = sum c x - 32 sum x ; codes carry 2^-24
            v = fmaf(d * (float)sc, fmaf(acc[k], 16777216.0f, -32.0f * X[k]), v);
        }
        return v;
    }
};

template <int FMT> struct FmtOf;
template <> struct FmtOf<RTA_Q4_K> { using T = Q4K; };
template <> struct FmtOf<RTA_Q6_K> { using T = Q6K; };

// The 64 x values of one slot and their per-run sums.
template <class F>
__device__ __forceinline__ void load_x(const float* __restrict__ xb, int slot, float xs[64], float X[F::kRuns]) {
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

// ------------------------------------------------------------ batch 1 ----
// x float4s each thread stages into LDS (at most).  Blocks are 256 threads (KW = 1, 2,
// 4: at most 4096, 8192, 16384 columns) or 192 (KW = 3: at most 12288), so cols / 4 is
// at most 4, 8, 16, 16 times blockDim.
constexpr int kXPerThread = 16;
__host__ __device__ constexpr int b1_lds_bytes(int slots) { return slots * 17 * 16; }

// KW waves per row task (cols = 64*64*KW at most); 256-thread blocks run 4/KW
// independent task groups when KW divides 4, otherwise one group of KW waves.
// R rows per lane per task (P*R rows per task).
template <int FMT, int R, int MODE, int KW>
__global__ void __launch_bounds__(256) gemv_b1_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                      const int64_t row_bytes, const int rows, const int cols,
                                                      const float* __restrict__ x, float* __restrict__ y,
                                                      float* __restrict__ partial, const int lpr, const int ntasks,
                                                      const float* __restrict__ nw, const float eps) {
    using F = typename FmtOf<FMT>::T;
    using Raw = typename F::Raw;
    constexpr bool kDual = MODE == kSwiglu;
    constexpr int kGroups = (KW == 3) ? 1 : 4 / KW;
    __shared__ float s_part[kGroups][KW][R][2][4];   // per wave partials (KW > 1), 4 subs max
    __shared__ float s_ss[4];                        // the fused RMSNorm's wave sums

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int group = wave / KW, wk = wave - group * KW;   // wave index inside its task group
    const int S = cols >> 6, P = kWave / lpr;
    const int sub = lane / lpr, lir = lane - sub * lpr;
    const int slot_i = wk * 64 + lir;
    const bool active = lir < lpr && slot_i < S && (KW == 1 || lpr == kWave);
    const int slot = active ? slot_i : 0;
    const int rpt = P * R;

    extern __shared__ float4 s_x[];   // slot s's 64 x values at float4 17 s (+1 pad: no bank conflicts)
    float xs[64], X[F::kRuns];
    const int stride = gridDim.x * kGroups;
    Raw bufA[R], bufB[R], bufA2[kDual ? R : 1], bufB2[kDual ? R : 1];

    // Every address is valid (inactive lanes read slot 0, rows clamp), so loads need no
    // guard: results of inactive lanes and of tasks past the end are discarded.
    auto load_task = [&](int t, Raw* dst, Raw* dst2) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(t * rpt + sub + P * r, rows - 1);  // clamped rows are discarded
            F::load(w + (int64_t)row * row_bytes, slot, dst[r]);
            if constexpr (kDual) F::load(w2 + (int64_t)row * row_bytes, slot, dst2[r]);
        }
    };

    // real == false: a task group past the end that only keeps the block's barriers
    // matched; it computes on stale registers and writes nothing.
    auto run_task = [&](int t, const Raw* src, const Raw* src2, bool real) {
        float acc[R], acc2[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = active ? F::slot_dot(src[r], slot, xs, X) : 0.0f;
            if constexpr (kDual) acc2[r] = active ? F::slot_dot(src2[r], slot, xs, X) : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = lane_group_sum<KW == 1>(acc[r], lpr);
            if constexpr (kDual) acc2[r] = lane_group_sum<KW == 1>(acc2[r], lpr);
        }
        if constexpr (KW > 1) {   // lpr == 64 here: one row pass per wave
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    s_part[group][wk][r][0][0] = acc[r];
                    if constexpr (kDual) s_part[group][wk][r][1][0] = acc2[r];
                }
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s = 0.0f, s2 = 0.0f;
#pragma unroll
                for (int k = 0; k < KW; ++k) {
                    s += s_part[group][k][r][0][0];
                    if constexpr (kDual) s2 += s_part[group][k][r][1][0];
                }
                acc[r] = s;
                if constexpr (kDual) acc2[r] = s2;
            }
            __syncthreads();
            if (wk != 0) return;
        }
        if (!real) return;
        float local_max = -INFINITY;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = t * rpt + sub + P * r;
            if (row >= rows) continue;
            const float v = acc[r];
            if constexpr (MODE == kLogits) local_max = fmaxf(local_max, v);
            if (lir == 0) {
                if constexpr (MODE == kStore || MODE == kLogits) y[row] = v;
                else if constexpr (MODE == kAccumulate) y[row] += v;
                else y[row] = swiglu(v, acc2[r]);
            }
        }
        if constexpr (MODE == kLogits) {
            local_max = max_across_groups(local_max, lpr);
            if (lane == 0) partial[t] = local_max;
        }
    };

    // Uniform trip count per block (KW > 1 groups synchronise inside run_task).
    // x goes through LDS: a lane's 64 values span 256 bytes, so direct per-lane loads
    // touch 64 cache lines per instruction.  The coalesced loads are issued first and
    // land in LDS while the first task's weights are in flight.
    // Loads and stores are unconditional, clamped to the last float4 (rewritten with its
    // own value): a guarded load becomes a branch that waits for it on the spot.
    constexpr int kXPer = KW == 1 ? 4 : KW == 2 ? 8 : kXPerThread;
    const int nf = cols >> 2;
    int xf[kXPer];
    float4 xg[kXPer];
#pragma unroll
    for (int k = 0; k < kXPer; ++k) {
        xf[k] = min((int)threadIdx.x + k * (int)blockDim.x, nf - 1);
        xg[k] = reinterpret_cast<const float4*>(x)[xf[k]];
    }
    const int task = blockIdx.x * kGroups + group;
    load_task(task, bufA, bufA2);
    // With nw, x is a residual row and the readout takes its RMSNorm (op 1): x w /
    // sqrt(mean(x^2) + eps), the sum of squares over the row's own float4s (clamped
    // duplicates excluded), per element in rmsnorm_kernel's order.
    if (nw) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < kXPer; ++k) {
            const float4 v = xg[k];
            if ((int)threadIdx.x + k * (int)blockDim.x < nf) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        // (a butterfly of shuffles: the DPP + row-swap sum here raised the register count of
        // the three-wave blocks past three waves per SIMD)
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
        if (lane == 0) s_ss[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += s_ss[i];
        const float inv = 1.0f / sqrtf(tot / (float)cols + eps);
#pragma unroll
        for (int k = 0; k < kXPer; ++k) {
            const float4 v = xg[k], g = reinterpret_cast<const float4*>(nw)[xf[k]];
            xg[k] = make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
        }
    }
#pragma unroll
    for (int k = 0; k < kXPer; ++k) {
        const int pl = F::place(4 * xf[k]);
        s_x[(pl >> 6) * 17 + ((pl & 63) >> 2)] = xg[k];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < F::kRuns; ++i) X[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 v = active ? s_x[slot * 17 + i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        xs[4 * i + 0] = v.x;
        xs[4 * i + 1] = v.y;
        xs[4 * i + 2] = v.z;
        xs[4 * i + 3] = v.w;
        X[(4 * i) / F::kRunLen] += (v.x + v.y) + (v.z + v.w);
    }
    for (int base = blockIdx.x * kGroups; base < ntasks; base += 2 * stride) {
        const int t0 = base + group, t1 = t0 + stride, t2 = t1 + stride;
        if (t1 < ntasks) load_task(t1, bufB, bufB2);
        if (t0 < ntasks) run_task(t0, bufA, bufA2, true);
        else if constexpr (KW > 1) run_task(t0, bufA, bufA2, false);
        if (base + stride >= ntasks) break;
        if (t2 < ntasks) load_task(t2, bufA, bufA2);
        if (t1 < ntasks) run_task(t1, bufB, bufB2, true);
        else if constexpr (KW > 1) run_task(t1, bufB, bufB2, false);
    }
}

// ------------------------------------------------------------ batch > 1 ----
// NB batch rows per launch; x slices are loaded per task (L1/L2 resident).
template <int FMT, int NB, int R, int MODE>
__global__ void __launch_bounds__(256) gemv_kquant_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                          const int64_t row_bytes, const int rows, const int cols,
                                                          const float* __restrict__ x, float* __restrict__ y,
                                                          float* __restrict__ partial, const int batch, const int lpr,
                                                          const int ntasks) {
    using F = typename FmtOf<FMT>::T;
    constexpr bool kDual = MODE == kSwiglu;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int S = cols >> 6;
    const int P = kWave / lpr;
    const int sub = lane / lpr, lir = lane - sub * lpr;
    const int ks = (S + lpr - 1) / lpr;
    const int rows_per_task = P * R;

    for (int task = blockIdx.x * 4 + wave; task < ntasks; task += gridDim.x * 4) {
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
                    const int row = min(row0 + P * r, rows - 1);   // clamped rows are discarded
                    F::load(w + (int64_t)row * row_bytes, slot, raw[r]);
                    if constexpr (kDual) F::load(w2 + (int64_t)row * row_bytes, slot, raw2[r]);
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    if (b < batch) {
                        float xs[64], X[F::kRuns];
                        load_x<F>(x + (int64_t)b * cols, slot, xs, X);
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            acc[r][b] += F::slot_dot(raw[r], slot, xs, X);
                            if constexpr (kDual) acc2[r][b] += F::slot_dot(raw2[r], slot, xs, X);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                acc[r][b] = lane_group_sum(acc[r][b], lpr);
                if constexpr (kDual) acc2[r][b] = lane_group_sum(acc2[r][b], lpr);
            }

        float local_max[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) local_max[b] = -INFINITY;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + P * r;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b >= batch || row >= rows) continue;
                float* out = y + (int64_t)b * rows + row;
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
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float m = local_max[b];
                m = max_across_groups(m, lpr);
                if (lane == 0 && b < batch) partial[(int64_t)b * ntasks + task] = m;
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
__global__ void __launch_bounds__(256) gemv_plain_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                                                         const int64_t row_bytes, const int rows, const int cols,
                                                         const float* __restrict__ x, float* __restrict__ y,
                                                         float* __restrict__ partial, const int batch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int row = blockIdx.x * 4 + wave; row < rows; row += gridDim.x * 4) {
        const uint8_t* wr = w + (int64_t)row * row_bytes;
        const uint8_t* wr2 = MODE == kSwiglu ? w2 + (int64_t)row * row_bytes : nullptr;
        for (int b = 0; b < batch; ++b) {
            const float* xb = x + (int64_t)b * cols;
            float s = 0.0f, s2 = 0.0f;
            for (int c = lane; c < cols; c += kWave) {
                s = fmaf(plain_value<FMT>(wr, c), xb[c], s);
                if constexpr (MODE == kSwiglu) s2 = fmaf(plain_value<FMT>(wr2, c), xb[c], s2);
            }
            s = lane_group_sum(s, kWave);
            if constexpr (MODE == kSwiglu) s2 = lane_group_sum(s2, kWave);
            if (lane == 0) {
                float* out = y + (int64_t)b * rows + row;
                if constexpr (MODE == kStore || MODE == kLogits) *out = s;
                else if constexpr (MODE == kAccumulate) *out += s;
                else *out = swiglu(s, s2);
                if constexpr (MODE == kLogits) partial[(int64_t)b * rows + row] = s;
            }
        }
    }
}

}  // namespace rta
