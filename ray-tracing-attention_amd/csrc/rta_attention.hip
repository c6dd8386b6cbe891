// rta_attention.hip -- split-K decode attention over quantised history packets,
// and rotary embedding (gfx950).
//
// The reference's detector (resident_ray.comp:56-76, ordered three-pass variant
// resident_detector_ordered_*.comp) walks every visible history slot -- its ray
// query returns all of them and checks the count (resident_ray.comp:30-53,80).
// Here the visible slots are enumerated in closed form, slot = base + p % capacity
// for p in [t+1-visible, t], and cut into 256-position chunks.  One workgroup
// handles one (sequence, kv head, chunk):
//   pass A  one lane per position: decode the position's K half-superblock once
//           and score it against the G query heads sharing that kv head (GQA);
//           chunk maximum m and Z = sum exp(s - m) per head.
//   pass B  eight position groups x 32 lanes of 4 coordinates: decode V once and
//           accumulate U[g] += w * V for all G heads; reduce the groups in LDS.
// A merge kernel combines the per-chunk (m, Z, U) records,
//   M = max m_c, Z = sum Z_c e^(m_c-M), o = sum U_c e^(m_c-M) / Z,
// which is the receipt merge of the grouped backends
// (resident_attention_runtime.inl:618-645).
#include <math.h>

#include "rta_common.hpp"
#include "rta_host.hpp"

namespace rta {

constexpr int kHd = 128;     // head dimension supported by these kernels
constexpr int kChunk = 256;  // positions per workgroup (the reference's tile, ordered_scores.comp:17)
constexpr int kRec = 2 + kHd; // per-head record: m, Z, U[128]

struct AttnArgs {
    const float* q;
    const uint8_t* packets;
    const int64_t* slot_base;
    const int32_t* ctx_len;
    const float* gate;
    float* out;
    float* m_out;
    float* z_out;
    float* ws;
    int64_t capacity;
    int64_t n_slots;    // packets in the array
    int64_t stride;     // packet bytes
    int64_t v_offset;   // byte offset of the V field inside a packet
    int nseq, hq, hkv, nchunk;
};

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Dword that starts at the 2-byte aligned address p (reads [floor4(p), floor4(p)+8)).
__device__ __forceinline__ uint32_t ld32_u2(const uint8_t* p) {
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t* w = reinterpret_cast<const uint32_t*>(p - mis);   // keeps the address space
    return mis ? funnel(w[0], w[1], mis) : w[0];
}

// ---- pass A: K scores ------------------------------------------------------
// Q4_K key half-superblock (head hh of the block): groups 4hh..4hh+3.
template <int G>
__device__ __forceinline__ void score_q4k(const uint8_t* blk, int hh, const float* __restrict__ qg,
                                          const float qs32[G][4], float score[G]) {
    const uint32_t h0 = ld32(blk), s0 = ld32(blk + 4), s1 = ld32(blk + 8), s2 = ld32(blk + 12);
    const float d = half_lo(h0), dmin = half_hi(h0);
#pragma unroll
    for (int g = 0; g < G; ++g) score[g] = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int jj = 2 * hh + u;
        const uint8_t* qsb = blk + 16 + 32 * jj;
        float alo[G], ahi[G];
#pragma unroll
        for (int g = 0; g < G; ++g) alo[g] = ahi[g] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t w = ld32(qsb + 4 * t), v = w >> 8;
            const half2_t p0 = as_codes(w & 0x000F000Fu), p1 = as_codes(v & 0x000F000Fu);
            const half2_t c0 = as_codes(w & 0x00F000F0u), c1 = as_codes(v & 0x00F000F0u);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float* qa = qg + g * kHd + 64 * u + 4 * t;
                alo[g] = fmaf((float)p0.x, qa[0], alo[g]);
                alo[g] = fmaf((float)p1.x, qa[1], alo[g]);
                alo[g] = fmaf((float)p0.y, qa[2], alo[g]);
                alo[g] = fmaf((float)p1.y, qa[3], alo[g]);
                ahi[g] = fmaf((float)c0.x, qa[32], ahi[g]);
                ahi[g] = fmaf((float)c1.x, qa[33], ahi[g]);
                ahi[g] = fmaf((float)c0.y, qa[34], ahi[g]);
                ahi[g] = fmaf((float)c1.y, qa[35], ahi[g]);
            }
        }
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(s0, s1, s2, 2 * jj, sc0, m0);
        q4k_scale_min(s0, s1, s2, 2 * jj + 1, sc1, m1);
        const float D0 = d * (float)sc0 * 16777216.0f, D1 = d * (float)sc1 * 1048576.0f;
        const float M0 = dmin * (float)m0, M1 = dmin * (float)m1;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float v2 = fmaf(D0, alo[g], score[g]);
            v2 = fmaf(-M0, qs32[g][2 * u], v2);
            v2 = fmaf(D1, ahi[g], v2);
            score[g] = fmaf(-M1, qs32[g][2 * u + 1], v2);
        }
    }
}

// Q6_K key half-superblock: dims l = 4t + 32k + e use ql byte 64hh + (l%64)
// (nibble l/64), qh byte 128 + 32hh + l%32 (bits 2(l/32)), scale 8hh + l/16.
template <int G>
__device__ __forceinline__ void score_q6k(const uint8_t* blk, int hh, const float* __restrict__ qg,
                                          const float qs16[G][8], float score[G]) {
    const float d = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(blk + 208));
    const uint32_t sc_lo = ld32_u2(blk + 192 + 8 * hh), sc_hi = ld32_u2(blk + 196 + 8 * hh);
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t a = ld32_u2(blk + 64 * hh + 4 * t), b = ld32_u2(blk + 64 * hh + 32 + 4 * t);
        const uint32_t h = ld32_u2(blk + 128 + 32 * hh + 4 * t);
        uint32_t c[4];
        c[0] = (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
        c[1] = (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
        c[2] = ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
        c[3] = ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const half2_t p = as_codes(c[k] & 0x00FF00FFu), r = as_codes((c[k] >> 8) & 0x00FF00FFu);
            const int grp = 2 * k + (t >> 2);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float* qa = qg + g * kHd + 32 * k + 4 * t;
                float v = acc[g][grp];
                v = fmaf((float)p.x, qa[0], v);
                v = fmaf((float)r.x, qa[1], v);
                v = fmaf((float)p.y, qa[2], v);
                v = fmaf((float)r.y, qa[3], v);
                acc[g][grp] = v;
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t sb = ((i < 4 ? sc_lo : sc_hi) >> (8 * (i & 3))) & 255u;
            const float D = d * (float)(int8_t)sb;
            s = fmaf(D, fmaf(acc[g][i], 16777216.0f, -32.0f * qs16[g][i]), s);
        }
        score[g] = s;
    }
}

// ---- pass B: V values for coordinates 4e..4e+3 of the head half -------------
__device__ __forceinline__ void values_q4k(const uint8_t* blk, int hh, int e, float v[4]) {
    const uint32_t h0 = ld32(blk);
    const int l = 4 * e, jj = 2 * hh + (l >> 6), hi = (l & 63) >> 5, g = 2 * jj + hi;
    uint32_t sc, m;
    q4k_scale_min(ld32(blk + 4), ld32(blk + 8), ld32(blk + 12), g, sc, m);
    const uint32_t w = ld32(blk + 16 + 32 * jj + (l & 31));
    const float D = half_lo(h0) * (float)sc, M = half_hi(h0) * (float)m;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = fmaf(D, (float)((w >> (8 * i + 4 * hi)) & 15u), -M);
}

__device__ __forceinline__ void values_q6k(const uint8_t* blk, int hh, int e, float v[4]) {
    const int l = 4 * e;
    const uint32_t a = ld32_u2(blk + 64 * hh + (l & 63));
    const uint32_t h = ld32_u2(blk + 128 + 32 * hh + (l & 31));
    const uint32_t sh = 8u * (uint32_t)((l >> 4) & 1);
    const uint32_t sb = ((uint32_t)*reinterpret_cast<const uint16_t*>(blk + 192 + 8 * hh + ((l >> 4) & ~1)) >> sh) & 255u;
    const float d = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(blk + 208));
    const float D = d * (float)(int8_t)sb;
    const uint32_t nib = (a >> (4 * (l >> 6))) & 0x0F0F0F0Fu;
    const uint32_t top = ((h >> (2 * (l >> 5))) & 0x03030303u) << 4;
    const uint32_t c = nib | top;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = D * (float)((int)((c >> (8 * i)) & 255u) - 32);
}

template <int KF, int VF, int G>
__global__ void __launch_bounds__(256) attn_chunk_kernel(const AttnArgs a) {
    __shared__ float s_w[kChunk][G];          // weights exp(s - m) per position
    __shared__ float s_red[4][G];
    __shared__ float s_u[8][G][kHd];          // per position-group partial U

    const int c = blockIdx.x, sk = blockIdx.y;
    const int s = sk / a.hkv, kvh = sk - s * a.hkv;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t L = a.ctx_len[s];
    const int64_t t = L - 1;
    const int64_t visible = L < a.capacity ? L : a.capacity;
    const int64_t first = (int64_t)c * kChunk;
    if (visible <= 0 || first >= visible) return;
    const int n = (int)(visible - first < kChunk ? visible - first : kChunk);
    const int64_t p0 = t + 1 - visible + first;     // oldest position of this chunk
    const int64_t base = a.slot_base[s];
    const int hh = kvh & 1;
    const int64_t kblk = (int64_t)(kvh >> 1) * (KF == RTA_Q4_K ? 144 : 210);
    const int64_t vblk = a.v_offset + (int64_t)(kvh >> 1) * (VF == RTA_Q4_K ? 144 : 210);
    const float* qg = a.q + ((int64_t)s * a.hq + (int64_t)kvh * G) * kHd;

    // Group sums of q used by the minimum / centring terms (uniform per wave).
    float qs32[G][4], qs16[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc += qg[g * kHd + 16 * i + e];
            qs16[g][i] = acc;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) qs32[g][i] = qs16[g][2 * i] + qs16[g][2 * i + 1];
    }

    // ---- pass A
    float score[G];
    bool live = tid < n;
    if (live) {
        const int64_t slot = base + (p0 + tid) % a.capacity;
        if (slot < 0 || slot >= a.n_slots) {
            raise_error(RTA_DEVERR_HITS);
            live = false;
        }
    }
    if (live) {
        const int64_t p = p0 + tid;
        const uint8_t* pk = a.packets + (base + p % a.capacity) * a.stride;
        if constexpr (KF == RTA_Q4_K) score_q4k<G>(pk + kblk, hh, qg, qs32, score);
        else score_q6k<G>(pk + kblk, hh, qg, qs16, score);
        const float inv = 1.0f / sqrtf((float)kHd);
        bool bad = false;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            score[g] *= inv;
            bad |= !isfinite(score[g]);
        }
        if (bad) raise_error(RTA_DEVERR_DETECTOR);
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) score[g] = -INFINITY;
    }
    float m[G], z[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float v = group_max(score[g], kWave);
        if (lane == 0) s_red[wave][g] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = fmaxf(fmaxf(s_red[0][g], s_red[1][g]), fmaxf(s_red[2][g], s_red[3][g]));
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float w = live ? expf(score[g] - m[g]) : 0.0f;
        s_w[tid][g] = w;
        const float v = group_sum(w, kWave);
        if (lane == 0) s_red[wave][g] = v;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) z[g] = (s_red[0][g] + s_red[1][g]) + (s_red[2][g] + s_red[3][g]);

    // ---- pass B
    const int grp = tid >> 5, e = tid & 31;
    float u[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) u[g][i] = 0.0f;
    for (int j = grp; j < n; j += 8) {
        const int64_t p = p0 + j;
        const int64_t slot = base + p % a.capacity;
        if (slot < 0 || slot >= a.n_slots) continue;   // flagged in pass A
        const uint8_t* pk = a.packets + slot * a.stride;
        float v[4];
        if constexpr (VF == RTA_Q4_K) values_q4k(pk + vblk, hh, e, v);
        else values_q6k(pk + vblk, hh, e, v);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float w = s_w[j][g];
#pragma unroll
            for (int i = 0; i < 4; ++i) u[g][i] = fmaf(w, v[i], u[g][i]);
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_u[grp][g][4 * e + i] = u[g][i];
    __syncthreads();
    float* rec = a.ws + ((int64_t)sk * a.nchunk + c) * G * kRec;
    for (int idx = tid; idx < G * kHd; idx += 256) {
        const int g = idx / kHd, dd = idx - g * kHd;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) acc += s_u[k][g][dd];
        rec[g * kRec + 2 + dd] = acc;
    }
    if (tid < G) {
        rec[tid * kRec + 0] = m[tid];
        rec[tid * kRec + 1] = z[tid];
    }
}

// One workgroup per (sequence, query head); thread = coordinate.
__global__ void __launch_bounds__(kHd) attn_merge_kernel(const AttnArgs a) {
    const int sh = blockIdx.x;
    const int s = sh / a.hq, h = sh - s * a.hq;
    const int G = a.hq / a.hkv, kvh = h / G, g = h - kvh * G;
    const int dd = threadIdx.x;
    const int64_t L = a.ctx_len[s];
    const int64_t visible = L < a.capacity ? L : a.capacity;
    float* out = a.out + (int64_t)sh * kHd;
    if (visible <= 0) {
        out[dd] = 0.0f;
        if (dd == 0) {
            if (a.m_out) a.m_out[sh] = -INFINITY;
            if (a.z_out) a.z_out[sh] = 0.0f;
            raise_error(RTA_DEVERR_HITS);
        }
        return;
    }
    int nch = (int)((visible + kChunk - 1) / kChunk);
    if (nch > a.nchunk) {  // max_ctx was below this sequence's visible count
        nch = a.nchunk;
        if (dd == 0) raise_error(RTA_DEVERR_HITS);
    }
    const float* rec0 = a.ws + ((int64_t)(s * a.hkv + kvh) * a.nchunk) * G * kRec + g * kRec;
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, rec0[(int64_t)c * G * kRec]);
    float Z = 0.0f, U = 0.0f;
    for (int c = 0; c < nch; ++c) {
        const float* rec = rec0 + (int64_t)c * G * kRec;
        const float f = expf(rec[0] - M);
        Z = fmaf(rec[1], f, Z);
        U = fmaf(rec[2 + dd], f, U);
    }
    float o = U / fmaxf(Z, 1e-30f);
    if (a.gate) o *= detector_sigmoid(a.gate[(int64_t)sh * kHd + dd]);
    out[dd] = o;
    if (dd == 0 && a.m_out) a.m_out[sh] = M;
    if (dd == 0 && a.z_out) a.z_out[sh] = Z;
}

// ---- RoPE -------------------------------------------------------------------
__global__ void __launch_bounds__(256) rope_kernel(float* __restrict__ v, int rows, int heads, int hd, int rotary,
                                                   const int64_t* __restrict__ positions, double theta) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2, active = rotary / 2;
    const int64_t total = (int64_t)rows * heads * half;
    if (i >= total) return;
    const int p = (int)(i % half);
    const int64_t rh = i / half;
    const int r = (int)(rh / heads);
    if (p >= active) return;
    const double phase = (double)positions[r] * pow(theta, -(double)p / (double)active);
    double sn, cs;
    sincos(phase, &sn, &cs);
    float* e = v + rh * hd + 2 * p;
    const double x = e[0], y = e[1];
    e[0] = (float)(x * cs - y * sn);
    e[1] = (float)(x * sn + y * cs);
}

template <int KF, int VF>
static hipError_t launch_chunks(int G, const AttnArgs& a, hipStream_t s) {
    const dim3 grid(a.nchunk, a.nseq * a.hkv);
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_chunk_kernel<KF, VF, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_chunk_kernel<KF, VF, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_chunk_kernel<KF, VF, 4>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((attn_chunk_kernel<KF, VF, 8>), grid, dim3(256), 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace rta

using namespace rta;

extern "C" {

int64_t rta_history_bytes(int kvw) { return host::history_bytes(kvw); }

int rta_rope(float* v, int rows, int heads, int hd, int rotary, const int64_t* positions, double theta,
             rta_stream_t stream) {
    if (!v || !positions) return RTA_ERR_NULL;
    if (rows <= 0 || heads <= 0 || hd <= 0 || hd % 2 || rotary < 0 || rotary > hd || rotary % 2) return RTA_ERR_SHAPE;
    if (!(theta > 0.0)) return RTA_ERR_RANGE;
    if (!host::aligned(v, 4) || !host::aligned(positions, 8)) return RTA_ERR_ALIGN;
    const int64_t total = (int64_t)rows * heads * (hd / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, v, rows,
                       heads, hd, rotary, positions, theta);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

size_t rta_decode_attention_workspace_bytes(int nseq, int hq, int hkv, int hd, int max_ctx) {
    if (nseq <= 0 || hq <= 0 || hkv <= 0 || hd != kHd || max_ctx <= 0 || hq % hkv) return 0;
    const int64_t nchunk = ((int64_t)max_ctx + kChunk - 1) / kChunk;
    return (size_t)nseq * (size_t)hkv * (size_t)nchunk * (size_t)(hq / hkv) * kRec * sizeof(float);
}

int rta_decode_attention(const float* q, int nseq, int hq, int hkv, int hd, const void* packets, int fmt_k, int fmt_v,
                         const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity, int64_t n_slots,
                         int max_ctx, const float* gate, float* out, float* m_out, float* z_out, void* workspace,
                         size_t workspace_bytes, rta_stream_t stream) {
    if (!q || !packets || !slot_base || !ctx_len || !out) return RTA_ERR_NULL;   // m_out, z_out optional
    if (nseq <= 0 || hq <= 0 || hkv <= 0 || hd <= 0 || hq % hkv || capacity <= 0 || max_ctx <= 0 || n_slots <= 0)
        return RTA_ERR_SHAPE;
    if ((fmt_k != RTA_Q4_K && fmt_k != RTA_Q6_K) || (fmt_v != RTA_Q4_K && fmt_v != RTA_Q6_K)) return RTA_ERR_FORMAT;
    const int G = hq / hkv;
    if (hd != kHd || (G != 1 && G != 2 && G != 4 && G != 8)) return RTA_ERR_RANGE;
    if (!host::aligned(q, 4) || !host::aligned(packets, 4) || !host::aligned(slot_base, 8) ||
        !host::aligned(ctx_len, 4) || !host::aligned(out, 4) || (gate && !host::aligned(gate, 4)))
        return RTA_ERR_ALIGN;
    const size_t need = rta_decode_attention_workspace_bytes(nseq, hq, hkv, hd, max_ctx);
    if (!workspace || workspace_bytes < need) return RTA_ERR_WORKSPACE;
    AttnArgs a{};
    a.q = q;
    a.packets = static_cast<const uint8_t*>(packets);
    a.slot_base = slot_base;
    a.ctx_len = ctx_len;
    a.gate = gate;
    a.out = out;
    a.m_out = m_out;
    a.z_out = z_out;
    a.ws = static_cast<float*>(workspace);
    a.capacity = capacity;
    a.n_slots = n_slots;
    const int kvw = hkv * kHd;
    a.stride = host::history_bytes(kvw);
    a.v_offset = (int64_t)((kvw + 255) / 256) * (fmt_k == RTA_Q4_K ? 144 : 210);
    a.nseq = nseq;
    a.hq = hq;
    a.hkv = hkv;
    a.nchunk = (int)((max_ctx + kChunk - 1) / kChunk);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (fmt_k == RTA_Q4_K && fmt_v == RTA_Q6_K) e = launch_chunks<RTA_Q4_K, RTA_Q6_K>(G, a, s);
    else if (fmt_k == RTA_Q6_K && fmt_v == RTA_Q4_K) e = launch_chunks<RTA_Q6_K, RTA_Q4_K>(G, a, s);
    else if (fmt_k == RTA_Q4_K) e = launch_chunks<RTA_Q4_K, RTA_Q4_K>(G, a, s);
    else e = launch_chunks<RTA_Q6_K, RTA_Q6_K>(G, a, s);
    if (e != hipSuccess) return RTA_ERR_LAUNCH;
    hipLaunchKernelGGL(attn_merge_kernel, dim3(nseq * hq), dim3(kHd), 0, s, a);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

}  // extern "C"
