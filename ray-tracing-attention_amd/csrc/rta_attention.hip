// rta_attention.hip -- split-K decode attention over quantised history packets,
// and rotary embedding (gfx950).
//
// The reference's detector (resident_ray.comp:56-76, ordered three-pass variant
// resident_detector_ordered_*.comp) walks every visible history slot -- its ray
// query returns all of them and checks the count (resident_ray.comp:30-53,80).
// Here the visible slots are enumerated in closed form, slot = base + p % capacity
// for p in [t+1-visible, t], and cut into chunks of nt tiles of 64 positions.
// One workgroup (4 waves) owns one (sequence, chunk) and every head of it, so each
// history packet is read from HBM by exactly one workgroup.  Per tile:
//   phase A  lane = position.  Each wave scores the K half-superblocks of its kv
//            heads against the G query heads sharing them (GQA); q stays uniform,
//            so the compiler keeps it in SGPRs and every code costs one
//            v_fma_mix_f32 per head.  In the same pass the lanes copy their
//            position's V superblocks into LDS (dword aligned), so the V loads are
//            in flight while the K arithmetic runs.
//   softmax  per head over the tile, folded into running (m, Z) with the online
//            rescale exp(m_old - m_new).
//   phase B  thread = (kv head, 16 or 8 coordinates, position group): V codes
//            from LDS, one v_fma_mix_f32 per code and head; the per-position
//            factor w * d * sc is applied once per sub-block run, and the Q4_K
//            minimum / Q6_K -32 offset is accumulated separately.
// Each chunk writes one (U[128], m, Z) record per head; a merge kernel combines
// them:  M = max m_c, Z = sum Z_c e^(m_c-M), o = sum U_c e^(m_c-M) / Z, which is the
// receipt merge of the grouped backends (resident_attention_runtime.inl:618-645).
#include <math.h>

#include <mutex>

#include "rta_common.hpp"
#include "rta_host.hpp"
#include "rta_internal.hpp"
#include "rta_pack.hpp"

namespace rta {

constexpr int kHd = 128;       // head dimension supported by these kernels
constexpr int kTile = 64;      // positions per tile: one per lane in phase A
constexpr int kRec = kHd + 4;  // per-head record: U[128], m, Z, 2 pad (16-byte multiple)
constexpr int kMaxLds = 160 * 1024;

struct AttnArgs {
    const float* q;
    const uint8_t* packets;
    const int64_t* slot_base;
    const int32_t* ctx_len;
    const float* gate;
    int64_t gate_stride;   // floats from one sequence's gate row to the next (head h at + h hd)
    int out_rotary;        // > 0: dim d < out_rotary of each head goes to column rot(d) of out
    float* out;
    float* m_out;
    float* z_out;
    float* ws;
    uint4* qop;         // matrix-core q operands [nseq][hkv][6][64] (Q4_K keys)
    int64_t capacity;
    int64_t n_slots;    // packets in the array
    int64_t stride;     // packet bytes
    int64_t v_offset;   // byte offset of the V field inside a packet
    int nseq, hq, hkv, nchunk;
    int nt;             // tiles per chunk
    int nblk;           // superblocks per field: ceil(hkv / 2)
    // tile-list split (matrix-core kernel): plan = [S[0..nseq]] tile prefix over the
    // sequences, then [nwg] the sequence holding each workgroup's first tile; records
    // [nseq][rstride][hq][kRec]; null for the chunk-grid kernels
    int32_t* plan;
    int nwg;
    int per_cu;         // workgroups resident on one compute unit (nwg = per_cu x compute units)
    bool prepared;      // q operands and plan already written (full_layer_middle)
    int64_t max_tiles;  // tiles per sequence at most: ceil(max_ctx / 64)
    int64_t rstride;    // records per sequence in the workspace
};
constexpr int kMaxWg = 2048;   // plan entries for workgroups

template <int FMT> struct Fmt;
template <> struct Fmt<RTA_Q4_K> { static constexpr int kBytes = 144, kRow = 37; };  // LDS row: 36 dwords + pad
template <> struct Fmt<RTA_Q6_K> { static constexpr int kBytes = 210, kRow = 53; };  // 52.5 dwords

// N consecutive dwords from a 4-byte aligned address, in 16-byte loads (each lane of a
// wave reads a different packet, so wide loads cut the cache-line requests per byte).
template <int N>
__device__ __forceinline__ void load_dwords(const uint32_t* __restrict__ p, uint32_t* r) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
        uint4 v;
        __builtin_memcpy(&v, p + 4 * i, 16);
        r[4 * i] = v.x;
        r[4 * i + 1] = v.y;
        r[4 * i + 2] = v.z;
        r[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = (N / 4) * 4; i < N; ++i) r[i] = p[i];
}

// LDS carve-up of the chunk kernel (dynamic shared memory), in floats.
// Phase B split: threads per kv head (128 coordinates, 16 or 8 per thread) and the
// number of position groups that share the workgroup's 256 threads.
__host__ __device__ constexpr int attn_tpk(int G) { return G == 8 ? 16 : 8; }
__host__ __device__ constexpr int attn_pg(int hkv, int G) { return 256 / (hkv * attn_tpk(G)); }

struct AttnLds {
    int m, z, scale, ok, qs, sc, w, v, total;
    __host__ __device__ AttnLds(int hq, int hkv, int nblk, int vrow) {
        m = 0;                        // [hq] running max
        z = m + hq;                   // [hq] running sum
        scale = z + hq;               // [hq] rescale of this tile
        ok = scale + hq;              // [64] position valid (int)
        qs = ok + kTile;              // [hq][8] 16-dim sums of q
        sc = (qs + hq * 8 + 3) & ~3;  // [hq][64] scores of the tile             } after the tiles:
        w = sc + hq * kTile;          // [hq][65] weights x 2^24 (padded)        } U partials
        v = (w + hq * (kTile + 1) + 3) & ~3;   // [nblk][64 vrow + 1] V superblocks } [PG][hq][128]
        const int vend = v + nblk * (kTile * vrow + 1);   // +1: superblock regions on different banks
        const int uend = sc + attn_pg(hkv, hq / hkv) * hq * kHd;
        total = vend > uend ? vend : uend;
    }
};

// Two binary16 sums in one v_pk_add_f16.
__device__ __forceinline__ uint32_t pk_add_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v_t, a) + __builtin_bit_cast(h2v_t, b));
}

// ---- phase A: K scores --------------------------------------------------------
// Q4_K key, head half hh of the superblock at blk (4-byte aligned).  Dims of the head:
// chunk jc (bytes 16 + 32(2hh+jc) ..), dword t: low nibbles are dims 64jc + 4t + b,
// high nibbles 64jc + 32 + 4t + b (resident_quant.glsl:10-15).
template <int G>
__device__ __forceinline__ void score_q4k(const uint8_t* __restrict__ blk, int hh, const float* __restrict__ qg,
                                          const float* qs, float score[G]) {
    const uint32_t* bw = reinterpret_cast<const uint32_t*>(blk);
    uint32_t hdr[4], w[16];
    load_dwords<4>(bw, hdr);
    load_dwords<16>(bw + 4 + 16 * hh, w);
    const float d = half_lo(hdr[0]), dmin = half_hi(hdr[0]);
#pragma unroll
    for (int g = 0; g < G; ++g) score[g] = 0.0f;
#pragma unroll
    for (int jc = 0; jc < 2; ++jc) {
        float alo[G], ahi[G];
#pragma unroll
        for (int g = 0; g < G; ++g) alo[g] = ahi[g] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t x = w[8 * jc + t], v = x >> 8;
            const half2_t p0 = as_codes(x & 0x000F000Fu), p1 = as_codes(v & 0x000F000Fu);
            const half2_t h0 = as_codes(x & 0x00F000F0u), h1 = as_codes(v & 0x00F000F0u);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float* qa = qg + g * kHd + 64 * jc + 4 * t;
                float a = alo[g], b = ahi[g];
                a = fmaf((float)p0.x, qa[0], a);
                a = fmaf((float)p1.x, qa[1], a);
                a = fmaf((float)p0.y, qa[2], a);
                a = fmaf((float)p1.y, qa[3], a);
                b = fmaf((float)h0.x, qa[32], b);
                b = fmaf((float)h1.x, qa[33], b);
                b = fmaf((float)h0.y, qa[34], b);
                b = fmaf((float)h1.y, qa[35], b);
                alo[g] = a;
                ahi[g] = b;
            }
        }
        const int jj = 2 * hh + jc;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(hdr[1], hdr[2], hdr[3], 2 * jj, sc0, m0);
        q4k_scale_min(hdr[1], hdr[2], hdr[3], 2 * jj + 1, sc1, m1);
        // low-nibble codes carry 2^-24, high-nibble codes 2^-20
        const float D0 = d * (float)sc0 * 16777216.0f, D1 = d * (float)sc1 * 1048576.0f;
        const float M0 = dmin * (float)m0, M1 = dmin * (float)m1;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float* qsg = qs + g * 8 + 4 * jc;
            float v2 = fmaf(D0, alo[g], score[g]);
            v2 = fmaf(-M0, qsg[0] + qsg[1], v2);
            v2 = fmaf(D1, ahi[g], v2);
            score[g] = fmaf(-M1, qsg[2] + qsg[3], v2);
        }
    }
}

// Q6_K key, head half hh of the superblock at blk (2-byte aligned).  Reads stay
// inside the 210-byte block: dwords from the 4-byte aligned address below, joined
// with alignbyte.  16-byte run c of ql (bytes 64hh + 16c ..) holds dims 16c + i in
// its low nibbles and 64 + 16c + i in its high nibbles; their two top bits come
// from qh bytes 128 + 32hh + 16(c & 1) + i at bit 2(c >> 1) and 2(2 + (c >> 1))
// (resident_quant.glsl:16-19).
template <int G>
__device__ __forceinline__ void score_q6k(const uint8_t* __restrict__ blk, int hh, const float* __restrict__ qg,
                                          const float* qs, float score[G]) {
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
    const uint32_t* a = reinterpret_cast<const uint32_t*>(blk - mis);
    uint32_t ql[17], qh[9], sw[2];
    load_dwords<17>(a + 16 * hh, ql);
    load_dwords<9>(a + 32 + 8 * hh, qh);
    __builtin_memcpy(sw, a + 48 + 2 * hh, 8);
    const uint32_t s0 = sw[0], s1 = sw[1];
    const uint32_t s2 = mis ? a[50 + 2 * hh] : s1;   // the third dword only exists when misaligned
    const uint32_t sc_lo = funnel(s0, s1, mis), sc_hi = funnel(s1, s2, mis);
    const float d = (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(blk + 208));
#pragma unroll
    for (int g = 0; g < G; ++g) score[g] = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float alo[G], ahi[G];
#pragma unroll
        for (int g = 0; g < G; ++g) alo[g] = ahi[g] = 0.0f;
        const uint32_t shl = 2u * (uint32_t)(c >> 1), shh = shl + 4u;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t A = funnel(ql[4 * c + t], ql[4 * c + t + 1], mis);
            const uint32_t H = funnel(qh[4 * (c & 1) + t], qh[4 * (c & 1) + t + 1], mis);
            const uint32_t lo = (A & 0x0F0F0F0Fu) | (((H >> shl) & 0x03030303u) << 4);
            const uint32_t hi = ((A >> 4) & 0x0F0F0F0Fu) | (((H >> shh) & 0x03030303u) << 4);
            // (c - 32) 2^-24 per code, exact binary16 subnormals: each element whole (a
            // -32 sum q term apart would cancel against the code term for small scores)
            const half2_t l0 = as_codes(pk_add_f16(lo & 0x00FF00FFu, 0x80208020u));
            const half2_t l1 = as_codes(pk_add_f16((lo >> 8) & 0x00FF00FFu, 0x80208020u));
            const half2_t h0 = as_codes(pk_add_f16(hi & 0x00FF00FFu, 0x80208020u));
            const half2_t h1 = as_codes(pk_add_f16((hi >> 8) & 0x00FF00FFu, 0x80208020u));
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float* qa = qg + g * kHd + 16 * c + 4 * t;
                float x = alo[g], y = ahi[g];
                x = fmaf((float)l0.x, qa[0], x);
                x = fmaf((float)l1.x, qa[1], x);
                x = fmaf((float)l0.y, qa[2], x);
                x = fmaf((float)l1.y, qa[3], x);
                y = fmaf((float)h0.x, qa[64], y);
                y = fmaf((float)h1.x, qa[65], y);
                y = fmaf((float)h0.y, qa[66], y);
                y = fmaf((float)h1.y, qa[67], y);
                alo[g] = x;
                ahi[g] = y;
            }
        }
        // sub-block scales c (low run) and 4 + c (high run) of this half
        const float Dl = d * (float)(int8_t)((sc_lo >> (8 * c)) & 255u);
        const float Dh = d * (float)(int8_t)((sc_hi >> (8 * c)) & 255u);
#pragma unroll
        for (int g = 0; g < G; ++g) {   // the codes carry 2^-24
            const float v = fmaf(Dl * 16777216.0f, alo[g], score[g]);
            score[g] = fmaf(Dh * 16777216.0f, ahi[g], v);
        }
    }
}

// ---- phase A on the matrix cores (K = Q4_K) --------------------------------------
// Per 16 positions and kv head, S^T = Q K^T with v_mfma_f32_16x16x32_f16:
//   A (16 x 32)  q: row 2g + part holds binary16 hi (part 0) / lo (part 1) of q_g * s_g,
//                s_g a power of two with max|q_g s_g| in [2^13, 2^14) (22 bits of q);
//   B (32 x 16)  K codes * sub-block scale as exact binary16 (a code c in the low
//                bits of a half is the subnormal c 2^-24; (c 2^-24)(sc 2^10) =
//                (16c 2^-24)(sc 2^6) = c sc 2^-14, c sc <= 945); column = position.
// k block kb (0..3) covers dims 64 (kb >> 1) + 32 (kb & 1) + [0, 32) of the head,
// i.e. Q4_K group 4 hh + kb; lane segment u holds k = 8u + perm[i] in slot i (the
// code-pair masks deliver dims (k, k + 2)).  A second MFMA takes the minimum term:
// A = 32-dim sums of q (scaled by s_g / 32) in slots kb, B = the 6-bit minimum codes.
// The lane that loads position p (column p % 16, segment u) receives its scores in
// output rows 4u .. 4u + 3: heads 2u and 2u + 1, hi and lo.
struct QOp {
    h8_t a[4];    // k blocks of q
    h8_t am;      // minimum-term operand (lanes of segment 0)
    float rs[2];  // 1 / s of heads 2u and 2u + 1
};

template <int G>
__device__ __forceinline__ QOp make_qop(const float* __restrict__ qg, int lane) {
    constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    const int row = lane & 15, g = row >> 1, part = row & 1, u = lane >> 4;
    const bool live = g < G;
    const float* qh = qg + (live ? g : 0) * kHd;
    float v[4][8], sum[4];
    float mx = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const float4* p = reinterpret_cast<const float4*>(qh + 64 * (kb >> 1) + 32 * (kb & 1) + 8 * u);
        const float4 x0 = p[0], x1 = p[1];
        const float t[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        sum[kb] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[kb][i] = live ? t[i] : 0.0f;
            mx = fmaxf(mx, fabsf(v[kb][i]));
            sum[kb] += v[kb][i];
        }
    }
    mx = max_xor32(max_xor16(mx));
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {   // fixed order: ((u0 + u1) + (u2 + u3))
        sum[kb] = add_xor32(add_xor16(sum[kb]));
    }
    const int e = operand_exponent(mx);
    const float sg = ldexpf(1.0f, 14 - e);
    QOp o;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = v[kb][perm[i]] * sg;
            const _Float16 hi = (_Float16)x;
            o.a[kb][i] = part ? (_Float16)(x - (float)hi) : hi;
        }
    }
    const _Float16 z = (_Float16)0.0f;
    o.am = h8_t{z, z, z, z, z, z, z, z};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const float x = sum[kb] * (sg * 0.03125f);
        const _Float16 hi = (_Float16)x;
        o.am[kb] = u == 0 ? (part ? (_Float16)(x - (float)hi) : hi) : z;
    }
    // rows 4u and 4u + 2 are heads 2u and 2u + 1 (their s lives in every segment)
    o.rs[0] = 1.0f / __shfl(sg, 4 * u, kWave);
    o.rs[1] = 1.0f / __shfl(sg, 4 * u + 2, kWave);
    return o;
}

// The tile list of the matrix-core kernel, built by one wave: sequence s holds tiles
// [S[s], S[s + 1]) (min(ceil(visible / 64), max_tiles) of them, the oldest positions
// first), and workgroup w of P = min(workgroups, T) takes tiles [floor(w T / P),
// floor((w + 1) T / P)), T = S[nseq], at least one.  Also records, per workgroup, the
// sequence holding its first tile: the workgroups whose first tile lies in s are w in
// [ceil(S[s] P / T), ceil(S[s + 1] P / T)).
__device__ __forceinline__ void attn_plan_wave(const AttnArgs& a) {
    const int lane = threadIdx.x & 63;
    auto tiles_of = [&](int s) {
        int64_t t = 0;
        if (s < a.nseq) {
            const int64_t L = a.ctx_len[s];
            const int64_t vis = L < a.capacity ? L : a.capacity;
            if (vis > 0) t = (vis + kTile - 1) / kTile;
            if (t > a.max_tiles) t = a.max_tiles;
        }
        return (int)t;
    };
    auto scan = [&](int t, int& before, int& total) {   // exclusive prefix over the wave
        int x = t;
        for (int off = 1; off < kWave; off <<= 1) {
            const int y = __shfl_up(x, off, kWave);
            if (lane >= off) x += y;
        }
        before = x - t;
        total = __shfl(x, kWave - 1, kWave);
    };
    int64_t T = 0;
    for (int s0 = 0; s0 < a.nseq; s0 += kWave) {
        int before, total;
        scan(tiles_of(s0 + lane), before, total);
        T += total;
    }
    int64_t carry = 0;
    const int64_t P = a.nwg < T ? a.nwg : T;   // workgroups in use: each gets a tile
    for (int s0 = 0; s0 < a.nseq; s0 += kWave) {
        const int s = s0 + lane;
        const int t = tiles_of(s);
        int before, total;
        scan(t, before, total);
        if (s < a.nseq) {
            const int64_t first = carry + before, end = first + t;
            a.plan[s] = (int32_t)first;
            if (T > 0 && t > 0) {
                for (int64_t w = (first * P + T - 1) / T; w < (end * P + T - 1) / T && w < P; ++w)
                    a.plan[a.nseq + 1 + w] = s;
            }
        }
        carry += total;
    }
    if (lane == 0) a.plan[a.nseq] = (int32_t)T;
}

// q operands of one (sequence, kv head), built once and read by every chunk: six
// 16-byte words per lane (a[0..3], am, rs).  With a plan (the matrix-core kernel), the
// extra block (hkv, 0) builds the tile list.
template <int G>
__global__ void __launch_bounds__(64) attn_qprep_kernel(const AttnArgs a) {
    const int kvh = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
    if (kvh == a.hkv) {
        if (s == 0 && a.plan) attn_plan_wave(a);
        return;
    }
    const QOp o = make_qop<G>(a.q + ((int64_t)s * a.hq + (int64_t)kvh * G) * kHd, lane);
    uint4* dst = a.qop + ((int64_t)s * a.hkv + kvh) * 6 * kWave + lane;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) dst[kb * kWave] = __builtin_bit_cast(uint4, o.a[kb]);
    dst[4 * kWave] = __builtin_bit_cast(uint4, o.am);
    dst[5 * kWave] = uint4{__builtin_bit_cast(uint32_t, o.rs[0]), __builtin_bit_cast(uint32_t, o.rs[1]), 0u, 0u};
}

__device__ __forceinline__ QOp load_qop(const uint4* __restrict__ src, int lane) {
    QOp o;
    src += lane;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) o.a[kb] = __builtin_bit_cast(h8_t, src[kb * kWave]);
    o.am = __builtin_bit_cast(h8_t, src[4 * kWave]);
    const uint4 r = src[5 * kWave];
    o.rs[0] = __builtin_bit_cast(float, r.x);
    o.rs[1] = __builtin_bit_cast(float, r.y);
    return o;
}

struct KRaw {        // one lane's share of a Q4_K key: header and its two 8-byte segments
    uint4 hdr;
    uint2 c[2];      // chunk 2hh + jc, bytes 8u .. 8u + 7
};

__device__ __forceinline__ void load_key_q4k(const uint8_t* __restrict__ blk, int hh, int u, KRaw& r) {
    __builtin_memcpy(&r.hdr, blk, 16);
#pragma unroll
    for (int jc = 0; jc < 2; ++jc) __builtin_memcpy(&r.c[jc], blk + 16 + 32 * (2 * hh + jc) + 8 * u, 8);
}

// Scores (times 1/sqrt(hd)) of the 16 positions of one key tile against the G heads of
// one kv head.  Returns them for heads 2u and 2u + 1 of this lane's position.
template <int G>
__device__ __forceinline__ void score_q4k_mma(const QOp& qo, const KRaw& r, int hh, int u, float inv,
                                              float out[2]) {
    uint32_t sc[4], mn[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) q4k_scale_min_lane(r.hdr.y, r.hdr.z, r.hdr.w, 4 * hh + kb, sc[kb], mn[kb]);
    f4_t D = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const uint2 c = r.c[kb >> 1];
        const uint32_t M = (kb & 1) ? 0x00F000F0u : 0x000F000Fu;
        const uint32_t sp = h2dup((float)sc[kb] * ((kb & 1) ? 64.0f : 1024.0f));
        const uint4 q4 = {pk_mul_f16(c.x & M, sp), pk_mul_f16((c.x >> 8) & M, sp), pk_mul_f16(c.y & M, sp),
                          pk_mul_f16((c.y >> 8) & M, sp)};
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(qo.a[kb], __builtin_bit_cast(h8_t, q4), D, 0, 0, 0);
    }
    const _Float16 z = (_Float16)0.0f;
    h8_t bm = h8_t{z, z, z, z, z, z, z, z};
    if (u == 0) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) bm[kb] = (_Float16)(float)mn[kb];
    }
    const f4_t Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(qo.am, bm, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    // sum_k (d sc c - dmin m) q = (d 2^14 (hi + lo) - dmin 2^5 (mhi + mlo)) / s
    const float dC = half_lo(r.hdr.x) * 16384.0f, dM = half_hi(r.hdr.x) * 32.0f;
#pragma unroll
    for (int eh = 0; eh < 2; ++eh)
        out[eh] = fmaf(dC, D[2 * eh] + D[2 * eh + 1], -dM * (Dm[2 * eh] + Dm[2 * eh + 1])) * qo.rs[eh] * inv;
}

// Scores of the two kv heads of one Q4_K superblock (head halves 0 and 1) in one output,
// for G <= 4: q0 holds kv head 0's q in A rows 0-7 (its rows 8-15 are zero, heads >= G),
// q1 kv head 1's in rows 8-15 (rows 0-7 zero), so that lane segment u receives heads
// 2 (u & 1) + eh of kv head u >> 1.  Both heads share the superblock's d and dmin.
__device__ __forceinline__ void score_q4k_mma_pair(const QOp& q0, const QOp& q1, const uint4 hdr, const uint2 c0[2],
                                                   const uint2 c1[2], int u, const float rs[2], float out[2]) {
    f4_t D = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const _Float16 z = (_Float16)0.0f;
    h8_t bm0 = h8_t{z, z, z, z, z, z, z, z}, bm1 = bm0;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const QOp& qo = hh ? q1 : q0;
        const uint2* c2 = hh ? c1 : c0;
        uint32_t sc[4], mn[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) q4k_scale_min_lane(hdr.y, hdr.z, hdr.w, 4 * hh + kb, sc[kb], mn[kb]);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const uint2 c = c2[kb >> 1];
            const uint32_t M = (kb & 1) ? 0x00F000F0u : 0x000F000Fu;
            const uint32_t sp = h2dup((float)sc[kb] * ((kb & 1) ? 64.0f : 1024.0f));
            const uint4 q4 = {pk_mul_f16(c.x & M, sp), pk_mul_f16((c.x >> 8) & M, sp), pk_mul_f16(c.y & M, sp),
                              pk_mul_f16((c.y >> 8) & M, sp)};
            D = __builtin_amdgcn_mfma_f32_16x16x32_f16(qo.a[kb], __builtin_bit_cast(h8_t, q4), D, 0, 0, 0);
        }
        if (u == 0) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) (hh ? bm1 : bm0)[kb] = (_Float16)(float)mn[kb];
        }
    }
    f4_t Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(q0.am, bm0, f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(q1.am, bm1, Dm, 0, 0, 0);
    const float dC = half_lo(hdr.x) * 16384.0f, dM = half_hi(hdr.x) * 32.0f;
#pragma unroll
    for (int eh = 0; eh < 2; ++eh)
        out[eh] = fmaf(dC, D[2 * eh] + D[2 * eh + 1], -dM * (Dm[2 * eh] + Dm[2 * eh + 1])) * rs[eh];
}

// Copies the V superblock at blk (2-byte aligned, `bytes` long) into an LDS row whose
// dword i holds block bytes 4i..4i+3.  Reads stay inside [blk, blk + bytes).
template <int FMT>
struct VStage {
    static constexpr int kRaw = (Fmt<FMT>::kBytes + 2 + 3) / 4;   // dwords covering a misaligned block
    uint32_t raw[kRaw];
    uint32_t mis;
    uint32_t tail;   // the block's last 2 bytes; the last word is chosen when stored, so
                     // that no arithmetic waits on the loads before they are needed
    __device__ __forceinline__ void load(const uint8_t* __restrict__ blk) {
        constexpr int kB = Fmt<FMT>::kBytes;
        mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);   // 0 or 2
        const uint32_t* a = reinterpret_cast<const uint32_t*>(blk - mis);
        tail = (uint32_t)*reinterpret_cast<const uint16_t*>(blk + kB - 2);
        // (kB + mis) / 4 whole dwords, then the last 2 bytes when (kB + mis) % 4 == 2
        load_dwords<kRaw - 1>(a, raw);
        if constexpr (FMT == RTA_Q6_K) {   // 52 + 2 bytes aligned; 53 dwords misaligned
            // the load is unconditional (a guarded load would wait on the spot); when
            // aligned it rereads an in-block dword and the tail is used instead
            raw[kRaw - 1] = a[mis ? kRaw - 1 : kRaw - 2];
        }
    }
    // raw word i, the last one resolved: Q4_K 36 dwords aligned, 36 + 2 bytes
    // misaligned; Q6_K 52 + 2 bytes aligned, 53 dwords misaligned
    __device__ __forceinline__ uint32_t word(int i) const {
        if (i < kRaw - 1) return raw[i];
        if constexpr (FMT == RTA_Q4_K) return mis ? tail : 0u;
        return mis ? raw[kRaw - 1] : tail;
    }
    __device__ __forceinline__ void store(uint32_t* row) const {
        constexpr int kOut = (Fmt<FMT>::kBytes + 3) / 4;
#pragma unroll
        for (int i = 0; i < kOut; ++i) row[i] = funnel(word(i), i + 1 < kRaw ? word(i + 1) : 0u, mis);
    }
};

// ---- phase B: V accumulation from an LDS row -----------------------------------
// Dims l0 .. l0 + DPT - 1 of head half hh, all inside one sub-block.  Returns the
// codes as DPT/4 dwords of bytes, and the sub-block factors: value = D * code - M.
template <int FMT, int DPT>
__device__ __forceinline__ void v_codes(const uint32_t* row, int hh, int l0, uint32_t c[DPT / 4], float& D,
                                        float& M) {
    if constexpr (FMT == RTA_Q4_K) {
        const int jj = 2 * hh + (l0 >> 6), hi = (l0 >> 5) & 1;
        const int base = 4 + 8 * jj + ((l0 & 31) >> 2);
#pragma unroll
        for (int k = 0; k < DPT / 4; ++k) c[k] = (row[base + k] >> (4 * hi)) & 0x0F0F0F0Fu;
        uint32_t sc, m;
        q4k_scale_min(row[1], row[2], row[3], 2 * jj + hi, sc, m);
        D = half_lo(row[0]) * (float)sc;
        M = half_hi(row[0]) * (float)m;
    } else {
        const int bl = (64 * hh + (l0 & 63)) >> 2, bh = (128 + 32 * hh + (l0 & 31)) >> 2;
        const uint32_t sl = 4u * (uint32_t)(l0 >> 6), sh = 2u * (uint32_t)(l0 >> 5);
#pragma unroll
        for (int k = 0; k < DPT / 4; ++k)
            c[k] = ((row[bl + k] >> sl) & 0x0F0F0F0Fu) | (((row[bh + k] >> sh) & 0x03030303u) << 4);
        const int si = 192 + 8 * hh + (l0 >> 4);
        const int sc = (int)(int8_t)((row[si >> 2] >> (8 * (si & 3))) & 255u);
        D = half_lo(row[52]) * (float)sc;
        M = 0.0f;
    }
}

// KPW > 0: K = Q4_K scored on the matrix cores, KPW (1 or 2) kv heads per wave
// (hkv <= 4 KPW); KPW == 0: scored on the vector ALUs, any hkv.
template <int KF, int VF, int G, int KPW>
__global__ void __launch_bounds__(256, 2) attn_chunk_kernel(const AttnArgs a) {
    static_assert(KPW == 0 || KF == RTA_Q4_K, "matrix-core scoring reads Q4_K keys");
    extern __shared__ __align__(16) float lds[];
    constexpr int TPK = attn_tpk(G);          // threads per kv head
    constexpr int DPT = kHd / TPK;            // phase B dims per thread
    constexpr int VROW = Fmt<VF>::kRow;
    const AttnLds L(a.hq, a.hkv, a.nblk, VROW);
    float* s_sc = lds + L.sc;
    float* s_w = lds + L.w;
    float* s_qs = lds + L.qs;
    float* s_m = lds + L.m;
    float* s_z = lds + L.z;
    float* s_scale = lds + L.scale;
    int* s_ok = reinterpret_cast<int*>(lds + L.ok);
    uint32_t* s_v = reinterpret_cast<uint32_t*>(lds + L.v);

    const int c = blockIdx.x, s = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hq = a.hq, hkv = a.hkv;
    const int64_t Lc = a.ctx_len[s];
    const int64_t visible = Lc < a.capacity ? Lc : a.capacity;
    const int64_t chunk = (int64_t)a.nt * kTile;
    const int64_t first = (int64_t)c * chunk;
    if (visible <= 0 || first >= visible) return;
    const int n_all = (int)(visible - first < chunk ? visible - first : chunk);
    const int64_t p0 = Lc - visible + first;   // oldest position of this chunk
    const int64_t base = a.slot_base[s];
    const float* qs_seq = a.q + (int64_t)s * hq * kHd;

    // prologue: 16-dim sums of q (the minimum / centring terms of vector-ALU scoring),
    // running (m, Z)
    for (int i = tid; i < (KPW > 0 ? 0 : hq * 8); i += 256) {
        const float* p = qs_seq + (int64_t)i * 16;
        float acc = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc += p[e];
        s_qs[i] = acc;
    }
    for (int h = tid; h < hq; h += 256) {
        s_m[h] = -INFINITY;
        s_z[h] = 0.0f;
    }
    __syncthreads();

    // phase B role
    const int kvl = hkv * TPK, PG = 256 / kvl;
    const int pg = tid / kvl, rr = tid - pg * kvl;
    const int bkvh = rr / TPK, part = rr - bkvh * TPK;
    const bool bact = pg < PG;
    const int l0 = part * DPT, bhh = bkvh & 1;
    float acc[G][DPT], off[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        off[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < DPT; ++i) acc[g][i] = 0.0f;
    }

    // q of this wave's kv heads as matrix-core operands, prepared by attn_qprep_kernel
    // (clamped heads are never used)
    QOp qo[KPW > 0 ? KPW : 1];
    if constexpr (KPW > 0) {
#pragma unroll
        for (int kl = 0; kl < KPW; ++kl)
            qo[kl] = load_qop(a.qop + ((int64_t)s * hkv + min(wave + 4 * kl, hkv - 1)) * 6 * kWave, lane);
    }

    // error bits are raised once at the end: a global atomic inside the loop would
    // keep the compiler from reading q through the scalar cache
    uint32_t err = 0;
    const float inv = 1.0f / sqrtf((float)kHd);
    const int ntile = (n_all + kTile - 1) / kTile;
    for (int tile = 0; tile < ntile; ++tile) {
        const int n = min(kTile, n_all - tile * kTile);
        // ---- phase A: lane = position j
        const int j = lane;
        bool ok = j < n;
        const uint8_t* pk = a.packets;
        if (ok) {
            const int64_t slot = base + (p0 + tile * kTile + j) % a.capacity;
            if (slot < 0 || slot >= a.n_slots) {
                err |= RTA_DEVERR_HITS;
                ok = false;
            } else {
                pk = a.packets + slot * a.stride;
            }
        }
        if (wave == 0) s_ok[j] = ok ? 1 : 0;
        VStage<VF> vst;
        const bool stage = ok && wave < a.nblk;
        if constexpr (KPW > 0) {
            // keys of the wave's kv heads for the 4 x 16 positions (lane: position
            // 16 rt + lane % 16, segment u), then this lane's V superblock; every
            // address is valid (invalid positions read slot 0, heads clamp)
            const int u = lane >> 4;
            const uint64_t pv = reinterpret_cast<uint64_t>(pk);
            const uint8_t* kp[4];
            bool okr[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const int src = 16 * rt + (lane & 15);
                const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)pv, src, kWave);
                const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(pv >> 32), src, kWave);
                kp[rt] = reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
                okr[rt] = __shfl(ok ? 1 : 0, src, kWave) != 0;
            }
            // order: V, first head's keys, V into LDS (V returns first), second head's
            // keys, then the scores; this keeps at most two key sets in registers
            vst.load(pk + a.v_offset + (int64_t)min(wave, a.nblk - 1) * Fmt<VF>::kBytes);
            KRaw kr[KPW][4];
            auto load_keys = [&](int kl) {
                const int kvh = min(wave + 4 * kl, hkv - 1);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
                    load_key_q4k(kp[rt] + (int64_t)(kvh >> 1) * Fmt<RTA_Q4_K>::kBytes, kvh & 1, u, kr[kl][rt]);
            };
            load_keys(0);
            if (stage) vst.store(s_v + (int64_t)wave * (kTile * VROW + 1) + j * VROW);
            if constexpr (KPW > 1) load_keys(1);
#pragma unroll
            for (int kl = 0; kl < KPW; ++kl) {
                const int kvh = wave + 4 * kl;
                if (kvh >= hkv) break;
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    float sc2[2];
                    score_q4k_mma<G>(qo[kl], kr[kl][rt], kvh & 1, u, inv, sc2);
#pragma unroll
                    for (int eh = 0; eh < 2; ++eh) {
                        const int g = 2 * u + eh;
                        if (g < G) {
                            if (okr[rt] && !isfinite(sc2[eh])) err |= RTA_DEVERR_DETECTOR;
                            s_sc[(kvh * G + g) * kTile + 16 * rt + (lane & 15)] = okr[rt] ? sc2[eh] : -INFINITY;
                        }
                    }
                }
            }
        } else {
        if (stage) vst.load(pk + a.v_offset + (int64_t)wave * Fmt<VF>::kBytes);
        for (int kvh = wave; kvh < hkv; kvh += 4) {
            float score[G];
            if (ok) {
                const float* qg = qs_seq + (int64_t)kvh * G * kHd;
                const uint8_t* kb = pk + (int64_t)(kvh >> 1) * Fmt<KF>::kBytes;
                if constexpr (KF == RTA_Q4_K) score_q4k<G>(kb, kvh & 1, qg, s_qs + kvh * G * 8, score);
                else score_q6k<G>(kb, kvh & 1, qg, s_qs + kvh * G * 8, score);
                bool bad = false;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    score[g] *= inv;
                    bad |= !isfinite(score[g]);
                }
                if (bad) err |= RTA_DEVERR_DETECTOR;
            } else {
#pragma unroll
                for (int g = 0; g < G; ++g) score[g] = -INFINITY;
            }
#pragma unroll
            for (int g = 0; g < G; ++g) s_sc[(kvh * G + g) * kTile + j] = score[g];
        }
        if (stage) vst.store(s_v + (int64_t)wave * (kTile * VROW + 1) + j * VROW);
        }
        for (int vb = wave + 4; vb < a.nblk; vb += 4) {   // more than 8 kv heads
            if (ok) {
                vst.load(pk + a.v_offset + (int64_t)vb * Fmt<VF>::kBytes);
                vst.store(s_v + (int64_t)vb * (kTile * VROW + 1) + j * VROW);
            }
        }
        __syncthreads();

        // ---- softmax of the tile, folded into the running (m, Z).  A wave takes heads
        // wave + 4i eight at a time so that their reductions interleave.
        for (int h0 = wave; h0 < hq; h0 += 32) {
            constexpr int kH = 8;
            float v[kH], mt[kH];
#pragma unroll
            for (int i = 0; i < kH; ++i) {
                const int h = h0 + 4 * i;
                v[i] = h < hq ? s_sc[h * kTile + lane] : -INFINITY;
            }
#pragma unroll
            for (int i = 0; i < kH; ++i) mt[i] = wave_max_dpp(v[i]);
            float w[kH], scale[kH], m_new[kH];
#pragma unroll
            for (int i = 0; i < kH; ++i) {
                const int h = h0 + 4 * i;
                const float m_old = h < hq ? s_m[h] : -INFINITY;
                m_new[i] = fmaxf(m_old, mt[i]);
                if (m_new[i] == -INFINITY) {
                    w[i] = 0.0f;
                    scale[i] = 1.0f;
                } else {
                    w[i] = expf(v[i] - m_new[i]);
                    scale[i] = expf(m_old - m_new[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < kH; ++i) {
                const int h = h0 + 4 * i;
                const float zt = wave_sum_dpp(w[i]);
                if (h < hq) {
                    s_w[h * (kTile + 1) + lane] = w[i] * 16777216.0f;
                    if (lane == 0) {
                        s_z[h] = s_z[h] * scale[i] + zt;
                        s_m[h] = m_new[i];
                        s_scale[h] = scale[i];
                    }
                }
            }
        }
        __syncthreads();

        // ---- phase B: U[g][l0 + i] += w * V over this group's positions
        if (bact) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float f = s_scale[bkvh * G + g];
                off[g] *= f;
#pragma unroll
                for (int i = 0; i < DPT; ++i) acc[g][i] *= f;
            }
            const uint32_t* vrows = s_v + (int64_t)(bkvh >> 1) * (kTile * VROW + 1);
            for (int jj = pg; jj < n; jj += PG) {
                if (!s_ok[jj]) continue;
                uint32_t cw[DPT / 4];
                float D, M;
                v_codes<VF, DPT>(vrows + jj * VROW, bhh, l0, cw, D, M);
                const float* wr = s_w + bkvh * G * (kTile + 1) + jj;
                // every element enters the sum whole, w D (c - mu) with value = D (c - mu):
                // a minimum (Q4_K, mu = M / D) or -32 offset (Q6_K) summed apart over the
                // history would cancel against the code term and lose the bits of small
                // results.  A Q4_K sub-block with D = 0 holds -M in every element; that
                // term goes to off.
                float wD[G], mu24 = 0.0f;
                if constexpr (VF == RTA_Q4_K) {
                    const bool dz = D == 0.0f;
                    mu24 = dz ? 0.0f : (M / D) * (1.0f / 16777216.0f);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const float wg = wr[g * (kTile + 1)];
                        wD[g] = wg * D;
                        if (dz) off[g] = fmaf(wg, M, off[g]);
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < G; ++g) wD[g] = wr[g * (kTile + 1)] * D;
                }
#pragma unroll
                for (int k = 0; k < DPT / 4; ++k) {
                    float e[4];   // (c - mu) 2^-24 of the four codes in dword k
                    if constexpr (VF == RTA_Q4_K) {
                        const half2_t lo = as_codes(cw[k] & 0x00FF00FFu), hi = as_codes((cw[k] >> 8) & 0x00FF00FFu);
                        e[0] = (float)lo.x - mu24;
                        e[1] = (float)hi.x - mu24;
                        e[2] = (float)lo.y - mu24;
                        e[3] = (float)hi.y - mu24;
                    } else {   // c 2^-24 - 32 2^-24, exact in binary16 (subnormals)
                        const half2_t lo = as_codes(pk_add_f16(cw[k] & 0x00FF00FFu, 0x80208020u));
                        const half2_t hi = as_codes(pk_add_f16((cw[k] >> 8) & 0x00FF00FFu, 0x80208020u));
                        e[0] = (float)lo.x;
                        e[1] = (float)hi.x;
                        e[2] = (float)lo.y;
                        e[3] = (float)hi.y;
                    }
#pragma unroll
                    for (int g = 0; g < G; ++g) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[g][4 * k + i] = fmaf(e[i], wD[g], acc[g][4 * k + i]);
                    }
                }
            }
        }
        __syncthreads();
    }

    // ---- combine the position groups and write the records.  Every group writes its
    // U to a slot of its own (over the scores, weights and V rows of the last tile);
    // after one barrier each thread adds the groups of its coordinates in group order.
    // Coordinates l0 + 4k + e (l0 = DPT part) sit at 4 (k TPK + part) + e, which keeps
    // the float4 stores free of bank conflicts.
    float* s_u = lds + L.sc;   // [PG][hq][128]
    // Q4_K: U = acc - 2^-24 sum w' M over the sub-blocks with D = 0 (off is 0 for Q6_K)
    const float corr = 1.0f / 16777216.0f;
    if (bact) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float* u = s_u + ((int64_t)pg * hq + bkvh * G + g) * kHd;
#pragma unroll
            for (int k = 0; k < DPT / 4; ++k)
                *reinterpret_cast<float4*>(u + 4 * (k * TPK + part)) =
                    float4{fmaf(-corr, off[g], acc[g][4 * k + 0]), fmaf(-corr, off[g], acc[g][4 * k + 1]),
                           fmaf(-corr, off[g], acc[g][4 * k + 2]), fmaf(-corr, off[g], acc[g][4 * k + 3])};
        }
    }
    __syncthreads();
    float* rec = a.ws + ((int64_t)s * a.nchunk + c) * hq * kRec;
    const int64_t gstride = (int64_t)hq * kHd;
    // two coordinates per thread and round, their loads issued together (the second is
    // clamped onto the first past the end)
    const int ncoord = hq * kHd;
    for (int i0 = tid; i0 < ncoord; i0 += 512) {
        float v[2];
        int dst[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int i = (i0 + 256 * t < ncoord) ? i0 + 256 * t : i0;
            const int h = i / kHd, dd = i - h * kHd;
            const int p = dd / DPT, k = (dd % DPT) >> 2, e = dd & 3;
            const float* src = s_u + h * kHd + 4 * (k * TPK + p) + e;
            dst[t] = h * kRec + dd;
            v[t] = src[0];
#pragma unroll 4
            for (int r = 1; r < PG; ++r) v[t] += src[r * gstride];
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) rec[dst[t]] = v[t];
    }
    for (int h = tid; h < hq; h += 256) {
        rec[h * kRec + kHd] = s_m[h];
        rec[h * kRec + kHd + 1] = s_z[h];
    }
    if (err) raise_error(err);
}

// ---- matrix-core attention for Q4_K keys and Q6_K values -------------------------
// One wave owns one K/V superblock of the (sequence, chunk): both of its kv heads
// (KPW = 2, hkv > 4), or one half of it (KPW = 1: kv head `wave`, superblock wave / 2),
// with all G query heads of each, from the loads through the scores, the softmax (in
// registers) and P V to the records, so the waves of a workgroup never wait for one
// another.  Per tile of 64 positions:
//   scores   S^T = Q K^T on the matrix cores (score_q4k_mma), lane = position in the
//            loads; the key header is read once for both halves.
//   staging  the lane's V superblock is written to the wave's LDS region transposed,
//            dword i of position p at [i][p], so that a lane reads one dword of 8
//            consecutive positions with two 16-byte reads.
//   softmax  per query head over the tile's 64 positions (4 per lane, 16-lane rows),
//            folded into the running (m, Z) held in registers.
//   P V      U^T = V^T P^T on the matrix cores, k = 32 positions per instruction:
//     A (16 x 32)  row r, position p: e = sc (c - 32), code times 8-bit sub-block
//                  scale (an integer, |e| <= 4096), as binary16 hi = f16(e) and
//                  lo = e - hi (exact: one fma), one instruction each.  Lane r reads
//                  ql dword r and qh dword r & 7 of the head half, which hold the
//                  codes of 8 dims per position: tile (b, nib), row r is head dim
//                  32 q + 4 (r & 7) + b with q = 2 nib + (r >= 8)
//                  (resident_quant.glsl:16-19).
//     B (32 x 16)  column 2g + part, position p: x = w_g(p) d(p) 2^S as binary16 hi
//                  (part 0) / lo (part 1): w the softmax weight exp(s - m), d the
//                  superblock scale, S a per-tile power of two with max |d| 2^S in
//                  [2^13, 2^14).
//     D (16 x 16)  row r, column 2g + part: sum_p e x, so U_g = (D_2g + D_2g+1) 2^-S.
//   The online rescale exp(m_old - m_new) 2^(S_new - S_old) is applied to D before
//   the tile's products.  The records are those of attn_chunk_kernel.
constexpr int kVtStride = kTile + 4;                        // dwords per transposed row
constexpr int kVtRows = (Fmt<RTA_Q6_K>::kBytes + 3) / 4;    // 53 dwords of a superblock
struct MmaWaveLds {                                         // one wave's region, dwords
    static constexpr int vt = 0;                            // [53][68] V, transposed
    static constexpr int w = kVtRows * kVtStride;           // [2][8][68] softmax weights
    static constexpr int f = w + 2 * 8 * kVtStride;         // [2][8] rescale factors
    static constexpr int total = f + 16;
};
static_assert(MmaWaveLds::w % 4 == 0 && MmaWaveLds::total % 4 == 0, "16-byte aligned rows");

// max / sum over the 16 lanes of each row (quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror)
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    return fmaxf(v, dpp_mov<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    return v + dpp_mov<0x140>(v);
}

// a * b - c with one rounding (v_pk_fma_f16 with a negated addend)
__device__ __forceinline__ uint32_t pk_fms_f16(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2v_t, a),
                                                                  __builtin_bit_cast(h2v_t, b),
                                                                  -__builtin_bit_cast(h2v_t, c)));
}

// NWV waves per workgroup: 4 (two workgroups per CU), or 8 with one kv head per wave
// (one workgroup per CU, when the whole tile list fits one tile per CU: each tile's
// serial work is then halved).
template <int G, int KPW, int NWV = 4>
__global__ void __launch_bounds__(64 * NWV, 2) attn_chunk_mma_kernel(const AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hkv = a.hkv;
    const int kv0 = KPW == 2 ? 2 * wave : wave;    // first kv head of the wave
    const int blk = KPW == 2 ? wave : wave >> 1;    // its K/V superblock
    if (kv0 >= hkv) return;                         // no workgroup barrier in this kernel
    const bool two = KPW == 2 && kv0 + 1 < hkv;     // uniform
    constexpr bool kPair = KPW == 2 && G <= 4;      // both kv heads' scores in one output
    // this workgroup's share [ta, tb) of the tile list, which runs through the
    // sequences in order (plan: S[s] = first tile of sequence s, S[nseq] = T, then the
    // sequence holding each workgroup's first tile)
    // (values read from memory that every lane shares are moved to scalar registers)
    auto uni = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    auto uni64 = [](int64_t v) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };
    const int32_t* S = a.plan;
    const int64_t T = uni(S[a.nseq]);
    const int64_t P = a.nwg < T ? a.nwg : T;   // every workgroup below P has a tile
    // v: this workgroup's place in the split.  With two workgroups per CU, workgroups b
    // and b + nwg / 2 are the two resident on one compute unit (dispatched in that
    // order), so they take adjacent shares and every compute unit gets floor or ceil of
    // 2 T / P tiles; the plain order would give both the same floor or ceil of T / P
    const int b = blockIdx.x, half = a.nwg / 2;
    const int64_t v = (a.per_cu == 2 && P == a.nwg && (a.nwg & 1) == 0) ? 2 * (b % half) + b / half : b;
    if (v >= P) return;   // (all of them when T = 0)
    const int64_t ta = v * T / P, tb = (v + 1) * T / P;
    int s = uni(S[a.nseq + 1 + v]);
    uint32_t* vt = reinterpret_cast<uint32_t*>(lds) + wave * MmaWaveLds::total;
    float* s_w = lds + wave * MmaWaveLds::total + MmaWaveLds::w;
    float* s_f = lds + wave * MmaWaveLds::total + MmaWaveLds::f;
    auto hh_of = [&](int kl) { return KPW == 2 ? kl : (wave & 1); };

    const int u = lane >> 4, col = lane & 15;   // row of 16 lanes, column in it

    // per-lane constants of the P V operands (A row r = col)
    const int qsel = col >= 8 ? 1 : 0;
    const uint32_t sbyte = (uint32_t)(((col & 7) >> 2) + 2 * qsel);   // sub-block scale byte
    const uint32_t sc_sel = sbyte | (0x0Cu << 8) | ((4u + sbyte) << 16) | (0x0Cu << 24);
    // qh bits 2q, 2q + 1 to bits 6, 7: rotate left by 6 - 2q (alignbit rotates right)
    const uint32_t rot[2] = {(32u - (uint32_t)((6 - 2 * qsel) & 31)) & 31u,
                             (32u - (uint32_t)((6 - 2 * (2 + qsel)) & 31)) & 31u};

    uint32_t err = 0;
    // scores in log2 units, s log2(e) / sqrt(hd), so that the softmax takes exp2 (one
    // v_exp_f32); m is converted back (times ln 2) for the records
    const float inv2 = 1.4426950408889634f / sqrtf((float)kHd);
    for (int64_t x = ta; x < tb;) {   // uniform: one sequence segment per pass
        const int64_t s_first = uni(S[s]), s_end = uni(S[s + 1]);
        if (s_end <= x) {
            ++s;
            continue;
        }
        const int64_t seg_end = s_end < tb ? s_end : tb;
        const int64_t base = uni64(a.slot_base[s]);     // both loads issued before either is used
        const int64_t Lc = uni(a.ctx_len[s]);
        const int64_t visible = Lc < a.capacity ? Lc : a.capacity;
        const int64_t n_vis = visible < a.max_tiles * kTile ? visible : a.max_tiles * kTile;
        // ring slot of sequence position off (< visible <= capacity): base + (p + off) %
        // capacity for the oldest visible position p, the modulo taken once
        const int64_t r0 = (Lc - visible) % a.capacity;
        float m_run[KPW][2], z_run[KPW][2];         // heads 2u + eh of each kv head
        f4_t D[KPW][8];
#pragma unroll
        for (int kl = 0; kl < KPW; ++kl) {
#pragma unroll
            for (int eh = 0; eh < 2; ++eh) {
                m_run[kl][eh] = -INFINITY;
                z_run[kl][eh] = 0.0f;
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) D[kl][t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
        int S_cur = 0;
        for (int64_t tile = x - s_first; tile < seg_end - s_first; ++tile) {
            const bool first_tile = tile == x - s_first;
            // the waves of the two workgroups on one compute unit share its SIMDs, whose
            // arbiter issues for the older wave first; they take turns at the higher
            // priority, tile by tile, so that neither runs its last tiles alone
            if (((int)tile ^ (b >= half ? 1 : 0)) & 1)
                __builtin_amdgcn_s_setprio(1);
            else
                __builtin_amdgcn_s_setprio(0);
            const int n = (int)(n_vis - tile * kTile < kTile ? n_vis - tile * kTile : kTile);
            // slot of the lane's position; past the tile's end the tile's last position
            // (its lines are read anyway), out of range slot 0
            const int j = lane;
            bool ok = j < n;
            int64_t slot;
            {
                const int64_t q = r0 + tile * kTile + min(j, n - 1);
                slot = base + (q >= a.capacity ? q - a.capacity : q);
            }
            if (slot < 0 || slot >= a.n_slots) {
                if (ok) err |= RTA_DEVERR_HITS;
                ok = false;
                slot = 0;
            }
            // V superblock first (it is needed first), then the keys of the 4 x 16
            // positions (lane: position 16 rt + col, segment u)
            VStage<RTA_Q6_K> vst;
            vst.load(a.packets + slot * a.stride + a.v_offset + (int64_t)blk * Fmt<RTA_Q6_K>::kBytes);
            uint4 hdr[4];
            uint2 kc[KPW][4][2];
            bool okr[4];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const int src = 16 * rt + col;
                const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)slot, src, kWave);
                const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)slot >> 32), src, kWave);
                okr[rt] = __shfl(ok ? 1 : 0, src, kWave) != 0;
                const uint8_t* kp = a.packets + (int64_t)(((uint64_t)hi << 32) | lo) * a.stride +
                                    (int64_t)blk * Fmt<RTA_Q4_K>::kBytes;
                __builtin_memcpy(&hdr[rt], kp, 16);
#pragma unroll
                for (int kl = 0; kl < KPW; ++kl)
#pragma unroll
                    for (int jc = 0; jc < 2; ++jc)
                        __builtin_memcpy(&kc[kl][rt][jc], kp + 16 + 32 * (2 * hh_of(kl) + jc) + 8 * u, 8);
            }
            // stage V transposed; the lane's d for the tile's scale 2^S
            float dabs;
            {
#pragma unroll
                for (int i = 0; i < kVtRows; ++i)
                    vt[i * kVtStride + j] = funnel(vst.word(i), i + 1 < VStage<RTA_Q6_K>::kRaw ? vst.word(i + 1) : 0u, vst.mis);
                dabs = ok ? fabsf(half_lo(funnel(vst.word(kVtRows - 1), 0u, vst.mis))) : 0.0f;
            }
            // q operands of the wave's kv heads (prepared by attn_qprep_kernel), reread per
            // tile from the cache once the V registers are free
            asm volatile("" ::: "memory");
            QOp qo[KPW];
            // paired scores (both kv heads in one output): kv head 1's operand rows move to
            // A rows 8-15 (lane - 8) and its 1 / s to segments 2, 3 (lane - 32)
            float rs_pair[2];
#pragma unroll
            for (int kl = 0; kl < KPW; ++kl) {
                const uint4* qsrc = a.qop + ((int64_t)s * hkv + min(kv0 + kl, hkv - 1)) * 6 * kWave;
                if (kPair && kl == 1) {
                    qo[kl] = load_qop(qsrc, col >= 8 ? lane - 8 : lane);
                    if (col < 8) {
                        const _Float16 z = (_Float16)0.0f;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb) qo[kl].a[kb] = h8_t{z, z, z, z, z, z, z, z};
                        qo[kl].am = h8_t{z, z, z, z, z, z, z, z};
                    }
                    const uint4 r = qsrc[5 * kWave + (u >= 2 ? lane - 32 : lane)];
                    // (qo[0].rs is already scaled by inv2)
                    rs_pair[0] = u >= 2 ? __builtin_bit_cast(float, r.x) * inv2 : qo[0].rs[0];
                    rs_pair[1] = u >= 2 ? __builtin_bit_cast(float, r.y) * inv2 : qo[0].rs[1];
                } else {
                    qo[kl] = load_qop(qsrc, lane);
                }
                qo[kl].rs[0] *= inv2;
                qo[kl].rs[1] *= inv2;
            }
            // scores of the wave's kv heads, heads 2u + eh, positions 16 rt + col (paired:
            // heads 2 (u & 1) + eh of kv head u >> 1, kept in sv[0])
            float sv[KPW][4][2];
            if constexpr (kPair) {
                const int klu = u >> 1, gu = 2 * (u & 1);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    float sc2[2];
                    score_q4k_mma_pair(qo[0], qo[1], hdr[rt], kc[0][rt], kc[1][rt], u, rs_pair, sc2);
#pragma unroll
                    for (int eh = 0; eh < 2; ++eh) {
                        const bool live = okr[rt] && gu + eh < G && (klu == 0 || two);
                        if (live && !isfinite(sc2[eh])) err |= RTA_DEVERR_DETECTOR;
                        sv[0][rt][eh] = live ? sc2[eh] : -INFINITY;
                    }
                }
            }
#pragma unroll
            for (int kl = 0; kl < KPW; ++kl) {
                if (kPair) break;
                if (kl == 1 && !two) break;
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    KRaw kr;
                    kr.hdr = hdr[rt];
                    kr.c[0] = kc[kl][rt][0];
                    kr.c[1] = kc[kl][rt][1];
                    float sc2[2];
                    score_q4k_mma<G>(qo[kl], kr, hh_of(kl), u, 1.0f, sc2);
#pragma unroll
                    for (int eh = 0; eh < 2; ++eh) {
                        const bool live = okr[rt] && 2 * u + eh < G;
                        if (live && !isfinite(sc2[eh])) err |= RTA_DEVERR_DETECTOR;
                        sv[kl][rt][eh] = live ? sc2[eh] : -INFINITY;
                    }
                }
            }
            // the power of two S: set on the first tile to put max |d| 2^S in [2^13, 2^14),
            // then kept while the tile's max |d| 2^S stays in [2^-4, 2^14) (no f16 overflow,
            // hi/lo still carrying 22 bits of the large terms), so D is rarely rescaled for it
            const float dmax = wave_max_dpp(dabs);
            int S_new = S_cur;
            if (dmax > 0.0f && isfinite(dmax)) {
                const float scaled = ldexpf(dmax, S_cur);
                if (first_tile || !(scaled < 16384.0f && scaled >= 0.0625f)) {
                    int e;
                    (void)frexpf(dmax, &e);
                    S_new = 14 - e;
                }
            }
            if (first_tile) S_cur = S_new;
            // softmax over the tile, folded into (m, Z); weights and rescale factors to LDS
            // (paired: one pass, lane segment u holding kv head u >> 1)
#pragma unroll
            for (int kl = 0; kl < (kPair ? 1 : KPW); ++kl) {
                if (kl == 1 && !two) break;
#pragma unroll
                for (int eh = 0; eh < 2; ++eh) {
                    const int klw = kPair ? (u >> 1) : kl;   // the kv head whose weights this lane writes
                    const int g = kPair ? 2 * (u & 1) + eh : 2 * u + eh;
                    const bool writes = g < G && (!kPair || klw == 0 || two);
                    float mx = fmaxf(fmaxf(sv[kl][0][eh], sv[kl][1][eh]), fmaxf(sv[kl][2][eh], sv[kl][3][eh]));
                    mx = row16_max(mx);
                    const float m_new = fmaxf(m_run[kl][eh], mx);
                    float w[4], sf;
                    if (m_new == -INFINITY) {
                        sf = 1.0f;
#pragma unroll
                        for (int rt = 0; rt < 4; ++rt) w[rt] = 0.0f;
                    } else {
                        sf = __builtin_amdgcn_exp2f(m_run[kl][eh] - m_new);
#pragma unroll
                        for (int rt = 0; rt < 4; ++rt) w[rt] = __builtin_amdgcn_exp2f(sv[kl][rt][eh] - m_new);
                    }
                    const float zt = row16_sum((w[0] + w[1]) + (w[2] + w[3]));
                    z_run[kl][eh] = z_run[kl][eh] * sf + zt;
                    m_run[kl][eh] = m_new;
                    if (writes) {
#pragma unroll
                        for (int rt = 0; rt < 4; ++rt) s_w[(klw * 8 + g) * kVtStride + 16 * rt + col] = w[rt];
                        if (col == 0) s_f[klw * 8 + g] = ldexpf(sf, S_new - S_cur);
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
            // rescale D (column 2g + part: head g), skipped when no running max and not S moved
            // (paired: columns 8 klc + 2g + part, kv head klc = col >> 3; each D[kl] is read
            // only in its own columns, so one factor per lane serves both)
            const int gcol = col >> 1;
            const int klc = kPair ? col >> 3 : 0, gp = kPair ? (col & 7) >> 1 : gcol;
            if constexpr (kPair) {
                const float fl = gp < G && (klc == 0 || two) ? s_f[klc * 8 + gp] : 1.0f;
                if (__builtin_amdgcn_ballot_w64(fl != 1.0f) != 0) {
#pragma unroll
                    for (int kl = 0; kl < KPW; ++kl)
#pragma unroll
                        for (int t = 0; t < 8; ++t) D[kl][t] *= fl;
                }
            }
#pragma unroll
            for (int kl = 0; kl < KPW; ++kl) {
                if (kPair) break;
                if (kl == 1 && !two) break;
                const float fl = gcol < G ? s_f[kl * 8 + gcol] : 1.0f;   // unused columns stay 0
                if (__builtin_amdgcn_ballot_w64(fl != 1.0f) != 0) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) D[kl][t] *= fl;
                }
            }
            S_cur = S_new;
            // P V, 32 positions per step: this lane's positions 32 ks + 8 u + i
#pragma unroll 1
            for (int ks = 0; ks < 2; ++ks) {
                const int pk0 = 32 * ks + 8 * u;
                float dS[8];
                {
                    const uint4 d0 = *reinterpret_cast<const uint4*>(vt + 52 * kVtStride + pk0);
                    const uint4 d1 = *reinterpret_cast<const uint4*>(vt + 52 * kVtStride + pk0 + 4);
                    const uint32_t dw[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) dS[i] = ldexpf(half_lo(dw[i]), S_cur);
                }
                // B: column col = head gcol, part col & 1 (paired: kv head col >> 3, head
                // (col & 7) >> 1, one operand for both): x = w d 2^S as hi + lo, both rounded
                // toward zero (|x - hi - lo| < 2^-21 |x|); columns of heads >= G are never read
                auto build_b = [&](int kl) {
                    h8_t bop;
                    {
                        const float* wr = s_w + (kPair ? klc * 8 + gp : kl * 8 + gcol) * kVtStride + pk0;
                        const float4 w0 = *reinterpret_cast<const float4*>(wr);
                        const float4 w1 = *reinterpret_cast<const float4*>(wr + 4);
                        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                        const bool part = (col & 1) != 0;
#pragma unroll
                        for (int i = 0; i < 8; i += 2) {
                            const float x0 = wv[i] * dS[i], x1 = wv[i + 1] * dS[i + 1];
                            const h2v_t h = __builtin_bit_cast(h2v_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
                            const h2v_t l =
                                __builtin_bit_cast(h2v_t, __builtin_amdgcn_cvt_pkrtz(x0 - (float)h.x, x1 - (float)h.y));
                            const h2v_t v = part ? l : h;
                            bop[i] = v.x;
                            bop[i + 1] = v.y;
                        }
                    }
                    return bop;
                };
                h8_t bop_pair;
                if constexpr (kPair) bop_pair = build_b(0);
#pragma unroll
                for (int kl = 0; kl < KPW; ++kl) {
                    if (kl == 1 && !two) break;
                    const int hh = hh_of(kl);
                    const h8_t bop = kPair ? bop_pair : build_b(kl);
                    // A: ql dword col, qh dword col & 7, sub-block scale dwords of nib 0 / 1
                    uint32_t ql[8], qh[8], sw[2][8];
                    {
                        auto rd8 = [&](int row, uint32_t* dst) {
                            const uint4 x0 = *reinterpret_cast<const uint4*>(vt + row * kVtStride + pk0);
                            const uint4 x1 = *reinterpret_cast<const uint4*>(vt + row * kVtStride + pk0 + 4);
                            dst[0] = x0.x; dst[1] = x0.y; dst[2] = x0.z; dst[3] = x0.w;
                            dst[4] = x1.x; dst[5] = x1.y; dst[6] = x1.z; dst[7] = x1.w;
                        };
                        rd8(16 * hh + col, ql);
                        rd8(32 + 8 * hh + (col & 7), qh);
                        rd8(48 + 2 * hh, sw[0]);
                        rd8(49 + 2 * hh, sw[1]);
                    }
                    // e 2^-14 = (c - 32) sc 2^-14, each element whole (a separate -32 sc term
                    // summed over the history would cancel against the code term and lose
                    // the bits of small results): the codes are built as 4 c in their bytes,
                    // so a code pair moved into 16-bit halves reads as c 2^-22 (binary16
                    // subnormals); minus 2^-17 that is (c - 32) 2^-22 (exact), and times
                    // sc 2^8 it gives (c - 32) sc 2^-14 as hi plus the exact remainder lo
                    // (|(c - 32) sc| <= 4096, every nonzero product >= 2^-14, so the
                    // matrix-core operands are normal); D is then in units of 2^(S - 14)
#pragma unroll
                    for (int nib = 0; nib < 2; ++nib) {
                        uint32_t code4[8], sc6[4];
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const uint32_t lo4 = nib ? (ql[i] >> 2) : (ql[i] << 2);
                            const uint32_t hi2 = __builtin_amdgcn_alignbit(qh[i], qh[i], rot[nib]) & 0xC0C0C0C0u;
                            code4[i] = (lo4 & 0x3C3C3C3Cu) | hi2;
                        }
#pragma unroll
                        for (int k = 0; k < 4; ++k) {   // int8 scales of positions 2k, 2k+1 as binary16
                            const uint32_t pr = __builtin_amdgcn_perm(sw[nib][2 * k + 1], sw[nib][2 * k], sc_sel);
                            const uint32_t sc = pk_add_f16((pr ^ 0x00800080u) | 0x64006400u, 0xE480E480u);   // - 1152
                            sc6[k] = pk_mul_f16(sc, 0x5C005C00u);    // sc 2^8
                        }
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const uint32_t sel = (uint32_t)b | (0x0Cu << 8) | ((4u + b) << 16) | (0x0Cu << 24);
                            uint32_t ah[4], al[4];
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const uint32_t cp = __builtin_amdgcn_perm(code4[2 * k + 1], code4[2 * k], sel);
                                const uint32_t cs = pk_add_f16(cp, 0x80808080u);   // - 2^-17 per half
                                ah[k] = pk_mul_f16(cs, sc6[k]);
                                al[k] = pk_fms_f16(cs, sc6[k], ah[k]);   // remainder, exact
                            }
                            const int t = 4 * nib + b;
                            D[kl][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                __builtin_bit_cast(h8_t, uint4{ah[0], ah[1], ah[2], ah[3]}), bop, D[kl][t], 0, 0, 0);
                            D[kl][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                __builtin_bit_cast(h8_t, uint4{al[0], al[1], al[2], al[3]}), bop, D[kl][t], 0, 0, 0);
                        }
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();   // the next tile's staging overwrites vt and s_w
        }

        // records: U_g[dim] = (D_2g + D_2g+1) 2^-S, then m and Z
        // record k of the sequence: k = this workgroup's place in the split - that of the
        // one holding its first tile
        const int64_t w_lo = ((s_first + 1) * P - 1) / T;
        float* rec = a.ws + ((int64_t)s * a.rstride + (v - w_lo)) * a.hq * kRec;
        const float unit = ldexpf(1.0f, 14 - S_cur);   // D is in units of 2^(S - 14)
        const int gcol = kPair ? (col & 7) >> 1 : col >> 1;   // the lane's head (paired: of kv head col >> 3)
#pragma unroll
        for (int kl = 0; kl < KPW; ++kl) {
            if (kl == 1 && !two) break;
            const bool writer = (col & 1) == 0 && gcol < G && (!kPair || (col >> 3) == kl);
            const int kvh = kv0 + kl;
            float* rh = rec + (int64_t)(kvh * G + (gcol < G ? gcol : 0)) * kRec;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int nib = t >> 2, b = t & 3;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = D[kl][t][e];
                    v += dpp_mov<0xB1>(v);                  // + the other part of the head
                    const int rr = 4 * u + e;
                    const int dim = 32 * (2 * nib + (rr >= 8 ? 1 : 0)) + 4 * (rr & 7) + b;
                    if (writer) rh[dim] = v * unit;
                }
            }
#pragma unroll
            for (int eh = 0; eh < 2; ++eh) {
                if (kPair) {   // lane segment u holds kv head u >> 1, heads 2 (u & 1) + eh
                    const int g = 2 * (u & 1) + eh, klw = u >> 1;
                    if (kl == 0 && col == 0 && g < G && (klw == 0 || two)) {
                        const int kvw = kv0 + klw;
                        rec[(int64_t)(kvw * G + g) * kRec + kHd] = m_run[0][eh] * 0.6931471805599453f;
                        rec[(int64_t)(kvw * G + g) * kRec + kHd + 1] = z_run[0][eh];
                    }
                } else {
                    const int g = 2 * u + eh;
                    if (col == 0 && g < G) {
                        rec[(int64_t)(kvh * G + g) * kRec + kHd] = m_run[kl][eh] * 0.6931471805599453f;
                        rec[(int64_t)(kvh * G + g) * kRec + kHd + 1] = z_run[kl][eh];
                    }
                }
            }
        }
        x = seg_end;
        ++s;
    }
    if (err) raise_error(err);
}

// ---- matrix-core attention for Q6_K keys and Q4_K values (hkv <= 4) ----------------
// attn_chunk_mma_kernel's structure (tile-list split, softmax in registers, the same
// records) for the other field pair, one kv head per wave.  Per tile of 64 positions:
//   scores   per 16 positions and k block of 32 dims (a quarter of the Q6_K head half):
//            A (16 x 32) q of the G heads as in score_q4k_mma (QOp, rows 2g + part hi /
//            lo), B (32 x 16) e = (c - 32) sc, column = position, lane segment u = dims
//            8u .. 8u + 7 of the quarter (one 16-dim sub-block, one scale); |e| <= 4096
//            is not always a binary16 integer, so B is its rounding hi plus the exact
//            remainder lo, one product each (score_q6k_mma).
//   P V      U^T = V^T P^T, k = 32 positions per instruction:
//            A (16 x 32) row r, position p: sc c of the Q4_K code (an integer <= 945,
//                        exact): qs dword r & 7 of chunk 2 hh + jc, nibble r >> 3, byte b,
//                        so a row's 8 positions share one sub-block 2 jc + (r >> 3);
//            B (32 x 16) column 2g + part: w_g(p) d(p) 2^S hi / lo as attn_chunk_mma_kernel;
//            the minimum term sum_p w dmin m 2^S takes one more product per 32
//            positions (A rows 0..3 = the head's 4 sub-blocks, 6-bit m; B = w dmin 2^S
//            hi / lo), and the record is U = (D - Dm of the dim's sub-block) 2^-S.  2^S
//            puts the tile's max(|d|, |dmin|) 2^S in [2^13, 2^14) (kept as in
//            attn_chunk_mma_kernel while it stays in [2^-4, 2^14)).
// The tile list in memory, for more sequences than one wave's lanes (one wave).
__global__ void __launch_bounds__(64) attn_plan_kernel(const AttnArgs a) { attn_plan_wave(a); }

// The tile list of attn_plan_wave for at most 64 sequences, held by a wave: lane s has
// sequence s's first tile and tile count, T the total.
struct WavePlan {
    int first, count;
    int64_t T;
};

__device__ __forceinline__ WavePlan wave_plan(const AttnArgs& a, int lane) {
    int t = 0;
    if (lane < a.nseq) {
        const int64_t L = a.ctx_len[lane];
        const int64_t vis = L < a.capacity ? L : a.capacity;
        int64_t n = vis > 0 ? (vis + kTile - 1) / kTile : 0;
        t = (int)(n > a.max_tiles ? a.max_tiles : n);
    }
    int x = t;
    for (int off = 1; off < kWave; off <<= 1) {
        const int y = __shfl_up(x, off, kWave);
        if (lane >= off) x += y;
    }
    return WavePlan{x - t, t, (int64_t)__shfl(x, kWave - 1, kWave)};
}

// One lane's share of a Q6_K key (head half hh of the superblock at sb, 2-byte
// aligned) for the products of k block kb = quarter kb of the half: elements r =
// 8u + i of each quarter (lane segment u).  Element l of the half is quarter l / 32,
// r = l % 32: ql byte 64 hh + 32 (quarter & 1) + r (high nibble for quarters 2, 3), qh
// byte 128 + 32 hh + r at bit 2 quarter, scale byte 192 + 8 hh + l / 16
// (resident_quant.glsl:16-19); the lane's 8 elements of a quarter share the scale of
// sub-block 2 kb + (u >> 1).  Reads stay inside the block: dwords from the aligned
// address below, joined with alignbyte.
struct K6Raw {
    uint32_t ql[4];   // ql bytes 64 hh + 8u .. + 7 (quarters 0, 2), 64 hh + 32 + 8u .. (1, 3)
    uint32_t qh[2];   // qh bytes 128 + 32 hh + 8u .. + 7
    uint32_t sc;      // byte kb: the int8 scale of sub-block 2 kb + (u >> 1)
    float d;
};

__device__ __forceinline__ void load_key_q6k(const uint8_t* __restrict__ sb, int hh, int u, K6Raw& r) {
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(sb) & 3u);
    const uint32_t* A = reinterpret_cast<const uint32_t*>(sb - mis);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = 16 * hh + 8 * k + 2 * u;
        const uint32_t a0 = A[i], a1 = A[i + 1], a2 = A[i + 2];
        r.ql[2 * k] = funnel(a0, a1, mis);
        r.ql[2 * k + 1] = funnel(a1, a2, mis);
    }
    {
        const int i = 32 + 8 * hh + 2 * u;
        const uint32_t a0 = A[i], a1 = A[i + 1], a2 = A[i + 2];
        r.qh[0] = funnel(a0, a1, mis);
        r.qh[1] = funnel(a1, a2, mis);
    }
    const uint32_t s0 = A[48 + 2 * hh], s1 = A[49 + 2 * hh], s2 = A[50 + 2 * hh];
    const uint32_t h = (uint32_t)(u >> 1);
    r.sc = __builtin_amdgcn_perm(funnel(s1, s2, mis), funnel(s0, s1, mis),
                                 h | ((2u + h) << 8) | ((4u + h) << 16) | ((6u + h) << 24));
    const uint32_t dw = A[52];   // bytes 208, 209 of the block
    r.d = mis ? half_hi(dw) : half_lo(dw);
}

// Scores (times 1 / 2^e, with qo.rs folded in) of the lane's position against heads 2u
// and 2u + 1 (rows 4u .. 4u + 3 of the output: head 2u hi, lo, head 2u + 1 hi, lo).
// B = (c - 32) sc, an integer of up to 4096 in magnitude, as binary16 hi (rounded) plus
// lo (the exact remainder, one fma), one product each.
__device__ __forceinline__ void score_q6k_mma(const QOp& qo, const K6Raw& r, float out[2]) {
    f4_t D = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        const uint32_t nsh = 4u * (uint32_t)(kb >> 1), hsh = 2u * (uint32_t)kb;
        uint32_t p[4];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t c = ((r.ql[2 * (kb & 1) + w] >> nsh) & 0x0F0F0F0Fu) |
                               (((r.qh[w] >> hsh) & 0x03030303u) << 4);
            // c - 32 as binary16: (1024 + c) - 1056, exact; pairs of elements (0, 2), (1, 3)
            p[2 * w] = pk_add_f16((c & 0x00FF00FFu) | 0x64006400u, 0xE420E420u);
            p[2 * w + 1] = pk_add_f16(((c >> 8) & 0x00FF00FFu) | 0x64006400u, 0xE420E420u);
        }
        const uint32_t sp = h2dup((float)(int8_t)((r.sc >> (8 * kb)) & 255u));
        uint32_t bh[4], bl[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            bh[k] = pk_mul_f16(p[k], sp);
            bl[k] = pk_fms_f16(p[k], sp, bh[k]);   // remainder, exact
        }
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(qo.a[kb], __builtin_bit_cast(h8_t, uint4{bh[0], bh[1], bh[2], bh[3]}),
                                                   D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(qo.a[kb], __builtin_bit_cast(h8_t, uint4{bl[0], bl[1], bl[2], bl[3]}),
                                                   D, 0, 0, 0);
    }
#pragma unroll
    for (int eh = 0; eh < 2; ++eh) out[eh] = r.d * (D[2 * eh] + D[2 * eh + 1]) * qo.rs[eh];
}

// The V rows a wave stages per position (transposed, [row][position]): row 0 the
// superblock's d | dmin, rows 1..4 its head half's sub-blocks 4 hh + l as binary16
// (sc | m << 16), rows 5..20 the half's 16 code dwords (chunks 2 hh, 2 hh + 1).
constexpr int kVt4Rows = 21;
struct Mma6WaveLds {                                   // one wave's region, dwords
    static constexpr int vt = 0;                       // [21][68] V, transposed
    static constexpr int w = kVt4Rows * kVtStride;     // [8][68] softmax weights
    static constexpr int f = w + 8 * kVtStride;        // [8] rescale factors
    static constexpr int q = f + 8;                    // [18][64] the segment's q operands
    static constexpr int total = q + 18 * kWave;
};
static_assert(Mma6WaveLds::w % 4 == 0 && Mma6WaveLds::total % 4 == 0, "16-byte aligned rows");
constexpr int kMma6LdsBytes = 4 * Mma6WaveLds::total * 4;

// The dwords of a Q4_K value superblock (at blk, 2-byte aligned) one head half needs:
// the header (d | dmin, 12 scale bytes) and the half's 16 code dwords.  An aligned block
// rereads an in-block dword instead of the one past it; a misaligned one (the only V
// superblock of a packet with one kv-head pair, at byte 210) reads its last dword
// whole, 2 bytes into the packet's padding to 8 bytes.
struct V4Half {
    uint32_t raw[22];
    uint32_t mis;
    __device__ __forceinline__ void load(const uint8_t* __restrict__ blk, int hh) {
        mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const uint32_t* A = reinterpret_cast<const uint32_t*>(blk - mis);
#pragma unroll
        for (int i = 0; i < 5; ++i) raw[i] = A[i];
#pragma unroll
        for (int i = 0; i < 16; ++i) raw[5 + i] = A[4 + 16 * hh + i];
        raw[21] = A[mis ? 20 + 16 * hh : 19 + 16 * hh];
    }
    __device__ __forceinline__ uint32_t hdr(int i) const { return funnel(raw[i], raw[i + 1], mis); }
    __device__ __forceinline__ uint32_t code(int i) const { return funnel(raw[5 + i], raw[6 + i], mis); }
};
constexpr int kMma6PerCu = 2;   // (registers admit two workgroups per compute unit)

template <int G>
__global__ void __launch_bounds__(256, 2) attn_chunk_mma6_kernel(const AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hkv = a.hkv;
    const int kvh = wave, blk = wave >> 1, hh = wave & 1;
    if (kvh >= hkv) return;   // no workgroup barrier in this kernel
    auto uni = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    auto uni64 = [](int64_t v) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };
    // the tile-list share and compute-unit pairing of attn_chunk_mma_kernel; the list
    // is built by every wave for at most 64 sequences (workgroup 0 leaves it in memory
    // for the merge), else read from memory
    const int32_t* S = a.plan;
    const bool in_reg = a.nseq <= kWave;
    WavePlan wp{0, 0, 0};
    if (in_reg) wp = wave_plan(a, lane);
    const int64_t T = in_reg ? wp.T : (int64_t)uni(S[a.nseq]);
    if (in_reg && blockIdx.x == 0 && wave == 0) {
        if (lane < a.nseq) a.plan[lane] = wp.first;
        if (lane == 0) a.plan[a.nseq] = (int32_t)T;
    }
    auto seq_first = [&](int q) { return in_reg ? (int64_t)uni(__shfl(wp.first, q, kWave)) : (int64_t)uni(S[q]); };
    auto seq_end = [&](int q) {
        return in_reg ? (int64_t)uni(__shfl(wp.first + wp.count, q, kWave)) : (int64_t)uni(S[q + 1]);
    };
    const int64_t P = a.nwg < T ? a.nwg : T;
    // (per_cu workgroups resident on one compute unit take adjacent shares)
    const int b = blockIdx.x, group = a.nwg / a.per_cu;
    const int64_t v = (P == a.nwg && a.nwg % a.per_cu == 0) ? a.per_cu * (b % group) + b / group : b;
    if (v >= P) return;
    const int64_t ta = v * T / P, tb = (v + 1) * T / P;
    int s;   // the sequence holding tile ta
    if (in_reg) {
        const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < a.nseq && wp.count > 0 && wp.first <= ta &&
                                                         ta < (int64_t)wp.first + wp.count);
        s = uni(hit ? (int)__builtin_ctzll(hit) : 0);
    } else {
        s = uni(S[a.nseq + 1 + v]);
    }
    uint32_t* vt = reinterpret_cast<uint32_t*>(lds) + wave * Mma6WaveLds::total;
    uint32_t* s_q = vt + Mma6WaveLds::q;
    float* s_w = lds + wave * Mma6WaveLds::total + Mma6WaveLds::w;
    float* s_f = lds + wave * Mma6WaveLds::total + Mma6WaveLds::f;
    const int u = lane >> 4, col = lane & 15;
    const int nib = col >> 3, gcol = col >> 1;
    uint32_t err = 0;
    const float inv2 = 1.4426950408889634f / sqrtf((float)kHd);   // scores in log2 units
    for (int64_t x = ta; x < tb;) {
        const int64_t s_first = seq_first(s), s_end = seq_end(s);
        if (s_end <= x) {
            ++s;
            continue;
        }
        const int64_t seg_end = s_end < tb ? s_end : tb;
        const int64_t base = uni64(a.slot_base[s]);
        const int64_t Lc = uni(a.ctx_len[s]);
        const int64_t visible = Lc < a.capacity ? Lc : a.capacity;
        const int64_t n_vis = visible < a.max_tiles * kTile ? visible : a.max_tiles * kTile;
        const int64_t r0 = (Lc - visible) % a.capacity;
        {   // the q operands of (s, kvh), kept in the wave's LDS for the segment
            const QOp o = make_qop<G>(a.q + ((int64_t)s * a.hq + (int64_t)kvh * G) * kHd, lane);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint4 w4 = __builtin_bit_cast(uint4, o.a[k]);
                s_q[(4 * k) * kWave + lane] = w4.x;
                s_q[(4 * k + 1) * kWave + lane] = w4.y;
                s_q[(4 * k + 2) * kWave + lane] = w4.z;
                s_q[(4 * k + 3) * kWave + lane] = w4.w;
            }
            s_q[16 * kWave + lane] = __builtin_bit_cast(uint32_t, o.rs[0] * inv2);
            s_q[17 * kWave + lane] = __builtin_bit_cast(uint32_t, o.rs[1] * inv2);
        }
        float m_run[2] = {-INFINITY, -INFINITY}, z_run[2] = {0.0f, 0.0f};
        f4_t D[8], Dm = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 8; ++t) D[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        int S_cur = 0;
        const int j = lane;
        // slot of the lane's position in a tile; past the tile's end its last position
        // (its lines are read anyway), out of range slot 0
        auto slot_of = [&](int64_t tile, bool& okp) {
            const int n = (int)(n_vis - tile * kTile < kTile ? n_vis - tile * kTile : kTile);
            okp = j < n;
            const int64_t q = r0 + tile * kTile + min(j, n - 1);
            int64_t sl = base + (q >= a.capacity ? q - a.capacity : q);
            if (sl < 0 || sl >= a.n_slots) {
                if (okp) err |= RTA_DEVERR_HITS;
                okp = false;
                sl = 0;
            }
            return sl;
        };
        auto v_block = [&](int64_t sl) {
            return a.packets + sl * a.stride + a.v_offset + (int64_t)blk * Fmt<RTA_Q4_K>::kBytes;
        };
        // keys of row rt of a tile (lane: position 16 rt + col, segment u) and whether
        // that position is valid
        auto load_row = [&](int rt, int64_t sl, bool okp, K6Raw& kr) {
            const int src = 16 * rt + col;
            const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)sl, src, kWave);
            const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)sl >> 32), src, kWave);
            const uint8_t* kp = a.packets + (int64_t)(((uint64_t)hi << 32) | lo) * a.stride +
                                (int64_t)blk * Fmt<RTA_Q6_K>::kBytes;
            load_key_q6k(kp, hh, u, kr);
            return __shfl(okp ? 1 : 0, src, kWave) != 0;
        };
        // the V superblock and first key row of a tile are loaded while the tile before
        // it is multiplied
        bool ok_next;
        int64_t slot_next = slot_of(x - s_first, ok_next);
        V4Half vst;
        vst.load(v_block(slot_next), hh);
        K6Raw k_first;
        bool ok_first = load_row(0, slot_next, ok_next, k_first);
        for (int64_t tile = x - s_first; tile < seg_end - s_first; ++tile) {
            const bool first_tile = tile == x - s_first;
            const bool ok = ok_next;
            const int64_t slot = slot_next;
            // the V superblock, staged transposed (the lane's max(|d|, |dmin|) for the
            // tile's 2^S); then the keys of the 4 x 16 positions (lane: position 16 rt +
            // col, segment u), each row's loads issued while the previous row is scored
            float dabs;
            {
                const uint32_t w0 = vst.hdr(0), h1 = vst.hdr(1), h2 = vst.hdr(2), h3 = vst.hdr(3);
                vt[j] = w0;
#pragma unroll
                for (int l = 0; l < 4; ++l) {   // (uniform sub-block: no lane select)
                    uint32_t sc, m;
                    q4k_scale_min(h1, h2, h3, 4 * hh + l, sc, m);
                    vt[(1 + l) * kVtStride + j] = pk_add_f16((sc | (m << 16)) | 0x64006400u, 0xE400E400u);
                }
#pragma unroll
                for (int c = 0; c < 16; ++c) vt[(5 + c) * kVtStride + j] = vst.code(c);
                dabs = ok ? fmaxf(fabsf(half_lo(w0)), fabsf(half_hi(w0))) : 0.0f;
            }
            bool okr[4];
            __builtin_amdgcn_sched_barrier(0);
            K6Raw kcur = k_first;
            okr[0] = ok_first;
            QOp qo;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                qo.a[k] = __builtin_bit_cast(h8_t, uint4{s_q[(4 * k) * kWave + lane], s_q[(4 * k + 1) * kWave + lane],
                                                         s_q[(4 * k + 2) * kWave + lane], s_q[(4 * k + 3) * kWave + lane]});
            qo.rs[0] = __builtin_bit_cast(float, s_q[16 * kWave + lane]);
            qo.rs[1] = __builtin_bit_cast(float, s_q[17 * kWave + lane]);
            float sv[4][2];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                float sc2[2];
                K6Raw knext;
                __builtin_amdgcn_sched_barrier(0);
                if (rt < 3) okr[rt + 1] = load_row(rt + 1, slot, ok, knext);
                score_q6k_mma(qo, kcur, sc2);
                kcur = knext;
#pragma unroll
                for (int eh = 0; eh < 2; ++eh) {
                    const bool live = okr[rt] && 2 * u + eh < G;
                    if (live && !isfinite(sc2[eh])) err |= RTA_DEVERR_DETECTOR;
                    sv[rt][eh] = live ? sc2[eh] : -INFINITY;
                }
            }
            const float dmax = wave_max_dpp(dabs);
            int S_new = S_cur;
            if (dmax > 0.0f && isfinite(dmax)) {
                const float scaled = ldexpf(dmax, S_cur);
                if (first_tile || !(scaled < 16384.0f && scaled >= 0.0625f)) {
                    int e;
                    (void)frexpf(dmax, &e);
                    S_new = 14 - e;
                }
            }
            if (first_tile) S_cur = S_new;
            // softmax over the tile, folded into (m, Z); weights and rescale factors to LDS
#pragma unroll
            for (int eh = 0; eh < 2; ++eh) {
                const int g = 2 * u + eh;
                float mx = fmaxf(fmaxf(sv[0][eh], sv[1][eh]), fmaxf(sv[2][eh], sv[3][eh]));
                mx = row16_max(mx);
                const float m_new = fmaxf(m_run[eh], mx);
                float w[4], sf;
                if (m_new == -INFINITY) {
                    sf = 1.0f;
#pragma unroll
                    for (int rt = 0; rt < 4; ++rt) w[rt] = 0.0f;
                } else {
                    sf = __builtin_amdgcn_exp2f(m_run[eh] - m_new);
#pragma unroll
                    for (int rt = 0; rt < 4; ++rt) w[rt] = __builtin_amdgcn_exp2f(sv[rt][eh] - m_new);
                }
                const float zt = row16_sum((w[0] + w[1]) + (w[2] + w[3]));
                z_run[eh] = z_run[eh] * sf + zt;
                m_run[eh] = m_new;
                if (g < G) {
#pragma unroll
                    for (int rt = 0; rt < 4; ++rt) s_w[g * kVtStride + 16 * rt + col] = w[rt];
                    if (col == 0) s_f[g] = ldexpf(sf, S_new - S_cur);
                }
            }
            __builtin_amdgcn_wave_barrier();
            {   // rescale D and Dm (column 2g + part: head g); unused columns stay 0
                const float fl = gcol < G ? s_f[gcol] : 1.0f;
                if (__builtin_amdgcn_ballot_w64(fl != 1.0f) != 0) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) D[t] *= fl;
                    Dm *= fl;
                }
            }
            S_cur = S_new;
            if (tile + 1 < seg_end - s_first) {   // the next tile's V and first key row, during P V
                slot_next = slot_of(tile + 1, ok_next);
                vst.load(v_block(slot_next), hh);
                ok_first = load_row(0, slot_next, ok_next, k_first);
            }
            // P V, 32 positions per step: this lane's positions 32 ks + 8 u + i
#pragma unroll 1
            for (int ks = 0; ks < 2; ++ks) {
                const int pk0 = 32 * ks + 8 * u;
                auto rd8 = [&](int row, uint32_t* dst) {
                    const uint4 x0 = *reinterpret_cast<const uint4*>(vt + row * kVtStride + pk0);
                    const uint4 x1 = *reinterpret_cast<const uint4*>(vt + row * kVtStride + pk0 + 4);
                    dst[0] = x0.x; dst[1] = x0.y; dst[2] = x0.z; dst[3] = x0.w;
                    dst[4] = x1.x; dst[5] = x1.y; dst[6] = x1.z; dst[7] = x1.w;
                };
                uint32_t hd8[8];
                rd8(0, hd8);
                // B: x = w f 2^S as hi + lo (f = d, or dmin for the minimum term), both
                // rounded toward zero; column col = head gcol, part col & 1
                auto build_b = [&](bool use_min) {
                    const float* wr = s_w + gcol * kVtStride + pk0;
                    const float4 w0 = *reinterpret_cast<const float4*>(wr);
                    const float4 w1 = *reinterpret_cast<const float4*>(wr + 4);
                    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                    const bool part = (col & 1) != 0;
                    h8_t bop;
#pragma unroll
                    for (int i = 0; i < 8; i += 2) {
                        const float f0 = ldexpf(use_min ? half_hi(hd8[i]) : half_lo(hd8[i]), S_cur);
                        const float f1 = ldexpf(use_min ? half_hi(hd8[i + 1]) : half_lo(hd8[i + 1]), S_cur);
                        const float x0 = wv[i] * f0, x1 = wv[i + 1] * f1;
                        const h2v_t h = __builtin_bit_cast(h2v_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
                        const h2v_t l =
                            __builtin_bit_cast(h2v_t, __builtin_amdgcn_cvt_pkrtz(x0 - (float)h.x, x1 - (float)h.y));
                        const h2v_t vv = part ? l : h;
                        bop[i] = vv.x;
                        bop[i + 1] = vv.y;
                    }
                    return bop;
                };
                const h8_t bop = build_b(false);
#pragma unroll
                for (int jc = 0; jc < 2; ++jc) {
                    // the row's sub-block 2 jc + nib of the half: sc of the 8 positions as
                    // binary16 pairs (the low halves of its staged row)
                    uint32_t scw[8], scp[4];
                    rd8(1 + 2 * jc + nib, scw);
#pragma unroll
                    for (int k = 0; k < 4; ++k) scp[k] = __builtin_amdgcn_perm(scw[2 * k + 1], scw[2 * k], 0x05040100u);
                    uint32_t qw[8];
                    rd8(5 + 8 * jc + (col & 7), qw);
#pragma unroll
                    for (int i = 0; i < 8; ++i) qw[i] = (qw[i] >> (4 * nib)) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) {
                        const uint32_t sel = (uint32_t)bb | (0x0Cu << 8) | ((4u + bb) << 16) | (0x0Cu << 24);
                        uint32_t ah[4];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t cp = __builtin_amdgcn_perm(qw[2 * k + 1], qw[2 * k], sel);
                            ah[k] = pk_mul_f16(pk_add_f16(cp | 0x64006400u, 0xE400E400u), scp[k]);   // sc c
                        }
                        const int t = 4 * jc + bb;
                        D[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(h8_t, uint4{ah[0], ah[1], ah[2], ah[3]}), bop, D[t], 0, 0, 0);
                    }
                }
                // the minimum term: A row r < 4 = the head's sub-block 4 hh + r (6-bit m)
                const h8_t bopm = build_b(true);
                uint32_t am[4];
                {
                    uint32_t mw[8];
                    rd8(1 + (col & 3), mw);   // (rows of lanes col >= 4 are zeroed)
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        am[k] = col < 4 ? __builtin_amdgcn_perm(mw[2 * k + 1], mw[2 * k], 0x07060302u) : 0u;
                }
                Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, uint4{am[0], am[1], am[2], am[3]}),
                                                            bopm, Dm, 0, 0, 0);
            }
            __builtin_amdgcn_wave_barrier();   // the next tile's staging overwrites vt and s_w
        }

        // records: U_g[dim] = (D - Dm of the dim's sub-block, both parts) 2^-S, then m, Z
        const int64_t w_lo = ((s_first + 1) * P - 1) / T;
        float* rec = a.ws + ((int64_t)s * a.rstride + (v - w_lo)) * a.hq * kRec;
        const float unit = ldexpf(1.0f, -S_cur);
        const bool writer = (col & 1) == 0 && gcol < G;
        float* rh = rec + (int64_t)(kvh * G + (gcol < G ? gcol : 0)) * kRec;
        float dm4[4];   // Dm rows 0..3 (sub-blocks) of this lane's column
#pragma unroll
        for (int e = 0; e < 4; ++e) dm4[e] = __shfl(Dm[e], col, kWave);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int jc = t >> 2, bb = t & 3;
            const int sbk = 2 * jc + (u >> 1);   // sub-block of rows 4u .. 4u + 3
            const float dm = sbk == 0 ? dm4[0] : sbk == 1 ? dm4[1] : sbk == 2 ? dm4[2] : dm4[3];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float val = D[t][e] - dm;
                val += dpp_mov<0xB1>(val);   // + the other part of the head
                const int rr = 4 * u + e;
                const int dim = 64 * jc + 32 * (rr >> 3) + 4 * (rr & 7) + bb;
                if (writer) rh[dim] = val * unit;
            }
        }
#pragma unroll
        for (int eh = 0; eh < 2; ++eh) {
            const int g = 2 * u + eh;
            if (col == 0 && g < G) {
                rec[(int64_t)(kvh * G + g) * kRec + kHd] = m_run[eh] * 0.6931471805599453f;
                rec[(int64_t)(kvh * G + g) * kRec + kHd + 1] = z_run[eh];
            }
        }
        x = seg_end;
        ++s;
    }
    if (err) raise_error(err);
}

// ---- the middle of a full-attention layer of the decode step --------------------------
// In-projection row r of sequence b = sum over k < nslab of proj[k slab_stride +
// b row_stride + r] in slab order (rows q | k | v | gate: hq, hkv, hkv and hq heads of
// 128).  Blocks (x, b), 256 threads:
//   x < nqb          query heads 4x .. 4x + 3, a wave each: QK-norm (op 14,
//                    resident_math.comp:113-114) and RoPE (op 3, resident_math.comp:76-77;
//                    phase resident_common.glsl:117; lane = the pair 2l, 2l + 1) to
//                    q_out; with qop the head's rows of its kv head's matrix-core q
//                    operands (make_qop's values); with a gate its summed rows to gate_out
//   x < nqb + nkv2   kv heads 2j, 2j + 1 (j = x - nqb): K norm and RoPE (waves 0, 1), V
//                    (waves 2, 3), then one superblock of each history field quantised by
//                    the packer routine rta_pack_history runs (pack_superblock_pair) and
//                    written to packet slot[b]; with kv_out the two rows as well
//   x == nqb + nkv2  (b = 0, with a plan) the attention's tile plan.
struct MiddleArgs {
    const float* proj;
    int64_t slab_stride;
    int row_stride, nslab, hq, hkv, G;
    const float *q_norm, *k_norm;
    float eps;
    const int64_t* positions;
    int rotary;
    double theta;
    float* q_out;
    uint4* qop;          // [nseq][hkv][6][64] or null
    float* gate_out;     // row b at gate_out + b gate_stride (head h at + 128 h), or null
    int64_t gate_stride;
    int fmt_k, fmt_v;
    const int64_t* slot;
    int64_t n_slots, stride, v_offset;
    uint8_t* packets;
    float* kv_out;       // [nseq][2][hkv 128]: the key and value rows quantised, or null
    int nqb, nkv2;
    AttnArgs plan;       // plan.plan null: no tile plan
};

template <int NS>
__global__ void __launch_bounds__(256) full_middle_kernel(const MiddleArgs p) {
    constexpr int hd = 128;
    __shared__ float xs[2][256];
    __shared__ float qsv[4][hd];
    __shared__ PackScratch st[2];
    __shared__ uint8_t fb[2][212];
    const int x = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float* src = p.proj + (int64_t)b * p.row_stride;
    auto load2 = [&](int r) {   // rows r, r + 1 summed over the slabs in slab order
        float2 t[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k)
            t[k] = *reinterpret_cast<const float2*>(src + (int64_t)min(k, p.nslab - 1) * p.slab_stride + r);
        float2 v = t[0];
#pragma unroll
        for (int k = 1; k < NS; ++k)
            if (k < p.nslab) {
                v.x += t[k].x;
                v.y += t[k].y;
            }
        return v;
    };
    // QK-norm and RoPE of the pair a lane holds, the phase and its sine / cosine in fp64
    auto norm_rope = [&](float2 v, const float* w) {
        if (w) {
            float ss = v.x * v.x + v.y * v.y;
            ss = wave_sum_dpp(ss);
            const float inv = 1.0f / sqrtf(ss / (float)hd + p.eps);
            v.x = v.x * inv * w[2 * lane];
            v.y = v.y * inv * w[2 * lane + 1];
        }
        const int active = p.rotary / 2;
        if (lane < active) {
            const double phase = (double)p.positions[b] * pow(p.theta, -(double)lane / (double)active);
            double sn, cs;
            sincos(phase, &sn, &cs);
            const double a0 = v.x, c0 = v.y;
            v.x = (float)(a0 * cs - c0 * sn);
            v.y = (float)(a0 * sn + c0 * cs);
        }
        return v;
    };
    if (x < p.nqb) {
        const int h = 4 * x + wave;
        if (h >= p.hq) return;   // uniform per wave; no block barrier below
        float2 v = load2(h * hd + 2 * lane);
        v = norm_rope(v, p.q_norm ? p.q_norm + h * hd : nullptr);
        *reinterpret_cast<float2*>(p.q_out + ((int64_t)b * p.hq + h) * hd + 2 * lane) = v;
        if (p.gate_out)
            *reinterpret_cast<float2*>(p.gate_out + (int64_t)b * p.gate_stride + h * hd + 2 * lane) =
                load2((p.hq + 2 * p.hkv + h) * hd + 2 * lane);
        if (!p.qop) return;
        // this head's rows 2g, 2g + 1 of its kv head's q operands (make_qop)
        const int G = p.G, kvh = h / G, g = h - kvh * G;
        qsv[wave][2 * lane] = v.x;
        qsv[wave][2 * lane + 1] = v.y;
        float mx = fmaxf(fabsf(v.x), fabsf(v.y));
        mx = wave_max_dpp(mx);
        const float sg = ldexpf(1.0f, 14 - operand_exponent(mx));
        __builtin_amdgcn_wave_barrier();
        uint4* dst = p.qop + ((int64_t)b * p.hkv + kvh) * 6 * kWave;
        const float* qv = qsv[wave];
        constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
        if (lane < 32) {   // word kb of lane (2g + part) + 16u
            const int part = lane & 1, u = (lane >> 1) & 3, kb = lane >> 3;
            const float* base = qv + 64 * (kb >> 1) + 32 * (kb & 1) + 8 * u;
            h8_t a;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float xv = base[perm[i]] * sg;
                const _Float16 hi = (_Float16)xv;
                a[i] = part ? (_Float16)(xv - (float)hi) : hi;
            }
            dst[kb * kWave + 2 * g + part + 16 * u] = __builtin_bit_cast(uint4, a);
        } else if (lane < 40) {   // the minimum-term word of lanes of segment 0
            const int part = lane & 1, u = (lane >> 1) & 3;
            const _Float16 z = (_Float16)0.0f;
            h8_t am = h8_t{z, z, z, z, z, z, z, z};
            if (u == 0) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    float s[4];   // (u0 + u1) + (u2 + u3), each the in-order sum of its 8 dims
#pragma unroll
                    for (int uu = 0; uu < 4; ++uu) {
                        const float* bb = qv + 64 * (kb >> 1) + 32 * (kb & 1) + 8 * uu;
                        float acc = 0.0f;
#pragma unroll
                        for (int i = 0; i < 8; ++i) acc += bb[i];
                        s[uu] = acc;
                    }
                    const float xv = ((s[0] + s[1]) + (s[2] + s[3])) * (sg * 0.03125f);
                    const _Float16 hi = (_Float16)xv;
                    am[kb] = part ? (_Float16)(xv - (float)hi) : hi;
                }
            }
            dst[4 * kWave + 2 * g + part + 16 * u] = __builtin_bit_cast(uint4, am);
        } else if (lane < 56) {   // 1 / s of this head in the rs word of segment g / 2
            float* rs = reinterpret_cast<float*>(dst + 5 * kWave + (lane - 40) + 16 * (g >> 1));
            rs[g & 1] = 1.0f / sg;
            if ((g & 1) == 0) {
                rs[2] = 0.0f;
                rs[3] = 0.0f;
            }
        }
        if (g == G - 1 && G < 8) {   // rows of heads >= G: zero operands, 1 / s = 2^-14
            const _Float16 z = (_Float16)0.0f;
            const uint4 zero = __builtin_bit_cast(uint4, h8_t{z, z, z, z, z, z, z, z});
            const int rows = 16 - 2 * G;
            for (int i = lane; i < rows * 4 * 5; i += kWave) {
                const int w = i / (rows * 4), rem = i - w * rows * 4;
                dst[w * kWave + 2 * G + rem % rows + 16 * (rem / rows)] = zero;
            }
            for (int gd = G + (G & 1); gd < 8; gd += 2)
                if (lane < 16) {
                    float* rs = reinterpret_cast<float*>(dst + 5 * kWave + lane + 16 * (gd >> 1));
                    rs[0] = 1.0f / 16384.0f;
                    rs[1] = 1.0f / 16384.0f;
                    rs[2] = 0.0f;
                    rs[3] = 0.0f;
                }
            if (G & 1 && lane < 16)   // the odd head count's partner: component 1 of segment G / 2
                reinterpret_cast<float*>(dst + 5 * kWave + lane + 16 * (G >> 1))[1] = 1.0f / 16384.0f;
        }
        return;
    }
    if (x < p.nqb + p.nkv2) {
        const int j = x - p.nqb;
        const int kh = 2 * j + (wave & 1);   // kv head of this wave
        const bool live = kh < p.hkv;       // uniform
        float2 v = float2{0.0f, 0.0f};
        if (wave < 2) {
            if (live) v = norm_rope(load2((p.hq + kh) * hd + 2 * lane), p.k_norm ? p.k_norm + kh * hd : nullptr);
            xs[0][(wave & 1) * hd + 2 * lane] = v.x;
            xs[0][(wave & 1) * hd + 2 * lane + 1] = v.y;
        } else {
            if (live) v = load2((p.hq + p.hkv + kh) * hd + 2 * lane);
            xs[1][(wave & 1) * hd + 2 * lane] = v.x;
            xs[1][(wave & 1) * hd + 2 * lane + 1] = v.y;
        }
        const bool q4[2] = {p.fmt_k == RTA_Q4_K, p.fmt_v == RTA_Q4_K};
        __syncthreads();
        if (p.kv_out) {   // the rows this block quantises: key then value row of sequence b
            const int kvw = p.hkv * hd, c = 256 * j + tid;
            if (c < kvw) {
                float* o = p.kv_out + (int64_t)b * 2 * kvw;
                o[c] = xs[0][tid];
                o[kvw + c] = xs[1][tid];
            }
        }
        pack_superblock_pair(xs, q4, st, fb, tid);
        const int64_t sl = p.slot[b];
        if (sl < 0 || sl >= p.n_slots) {
            if (tid == 0) raise_error(RTA_DEVERR_HITS);
            return;
        }
        uint8_t* pk = p.packets + sl * p.stride;
        const int kb = q4[0] ? 144 : 210, vb = q4[1] ? 144 : 210;
        for (int i = tid; i < kb; i += 256) pk[(int64_t)j * kb + i] = fb[0][i];
        for (int i = tid; i < vb; i += 256) pk[p.v_offset + (int64_t)j * vb + i] = fb[1][i];
        if (j == 0) {   // the packet's padding
            const int64_t end = p.v_offset + (int64_t)p.nkv2 * vb;
            for (int64_t i = end + tid; i < p.stride; i += 256) pk[i] = 0;
        }
        return;
    }
    if (b == 0 && wave == 0 && p.plan.plan) attn_plan_wave(p.plan);
}

// One workgroup per (sequence, query head): 8 chunk groups x 32 lanes of 4
// coordinates; every thread keeps 8 chunk records in flight.  One pass: each group
// folds its records into a running (m, Z, U), rescaled when m grows, and the groups
// are combined at the end (the same sums as max-then-accumulate, in another order).
// GROUPS groups of 32 threads, kAhead records in flight per group: 16 (512 threads) when
// a sequence's records can number in the hundreds (few sequences share the grid), else 8.
template <int GROUPS>
__global__ void __launch_bounds__(32 * GROUPS) attn_merge_kernel(const AttnArgs a) {
    constexpr int kGroups = GROUPS, kAhead = 8;
    __shared__ float4 s_u[kGroups][kHd / 4];
    __shared__ float s_zp[kGroups], s_mp[kGroups];
    const int sh = blockIdx.x;
    const int s = sh / a.hq, h = sh - s * a.hq;
    const int tid = threadIdx.x;
    const int grp = tid >> 5, e = tid & 31;
    const int64_t L = a.ctx_len[s];
    const int64_t visible = L < a.capacity ? L : a.capacity;
    float* out = a.out + (int64_t)sh * kHd;
    if (visible <= 0) {
        if (tid < kHd) out[tid] = 0.0f;
        if (tid == 0) {
            if (a.m_out) a.m_out[sh] = -INFINITY;
            if (a.z_out) a.z_out[sh] = 0.0f;
            raise_error(RTA_DEVERR_HITS);
        }
        return;
    }
    const int64_t cstride = (int64_t)a.hq * kRec;
    int nch;
    bool short_grid;   // max_ctx was below this sequence's visible count
    const float* rec0;
    if (a.plan) {   // one record per workgroup that covered tiles of the sequence
        const int64_t T = a.plan[a.nseq], P = a.nwg < T ? a.nwg : T;
        const int64_t first = a.plan[s], end = a.plan[s + 1];
        nch = (int)(((end * P - 1) / T) - (((first + 1) * P - 1) / T) + 1);
        short_grid = visible > a.max_tiles * kTile;
        rec0 = a.ws + (int64_t)s * a.rstride * cstride + (int64_t)h * kRec;
    } else {        // one record per chunk
        const int64_t chunk = (int64_t)a.nt * kTile;
        nch = (int)((visible + chunk - 1) / chunk);
        short_grid = nch > a.nchunk;
        if (short_grid) nch = a.nchunk;
        rec0 = a.ws + (int64_t)s * a.nchunk * cstride + (int64_t)h * kRec;
    }
    float Mg = -INFINITY, Z = 0.0f;   // the group's running max, sum and vector
    float4 U = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    {
        for (int c0 = grp; c0 < nch; c0 += kGroups * kAhead) {
            float mm[kAhead], zz[kAhead];
            float4 uu[kAhead];
#pragma unroll
            for (int k = 0; k < kAhead; ++k) {
                const int ci = c0 + kGroups * k;
                if (ci < nch) {
                    const float* r = rec0 + (int64_t)ci * cstride;
                    mm[k] = r[kHd];
                    zz[k] = r[kHd + 1];
                    uu[k] = *reinterpret_cast<const float4*>(r + 4 * e);
                } else {
                    mm[k] = -INFINITY;
                    zz[k] = 0.0f;
                    uu[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
            }
            float mb = Mg;
#pragma unroll
            for (int k = 0; k < kAhead; ++k) mb = fmaxf(mb, mm[k]);
            if (mb != -INFINITY) {   // uniform over the group's lanes
                if (mb != Mg) {
                    const float r = Mg == -INFINITY ? 0.0f : expf(Mg - mb);
                    Z *= r;
                    U.x *= r;
                    U.y *= r;
                    U.z *= r;
                    U.w *= r;
                    Mg = mb;
                }
            }
#pragma unroll
            for (int k = 0; k < kAhead; ++k) {
                const float f = mm[k] == -INFINITY ? 0.0f : expf(mm[k] - Mg);
                Z = fmaf(zz[k], f, Z);
                U.x = fmaf(uu[k].x, f, U.x);
                U.y = fmaf(uu[k].y, f, U.y);
                U.z = fmaf(uu[k].z, f, U.z);
                U.w = fmaf(uu[k].w, f, U.w);
            }
        }
    }
    s_u[grp][e] = U;
    if (e == 0) {
        s_zp[grp] = Z;
        s_mp[grp] = Mg;
    }
    __syncthreads();
    if (tid < kHd) {
        float M = -INFINITY;
#pragma unroll
        for (int g = 0; g < kGroups; ++g) M = fmaxf(M, s_mp[g]);
        float u = 0.0f, z = 0.0f;
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            const float f = s_mp[g] == -INFINITY ? 0.0f : expf(s_mp[g] - M);
            u = fmaf(reinterpret_cast<const float*>(&s_u[g][0])[tid], f, u);
            z = fmaf(s_zp[g], f, z);
        }
        float o = u / fmaxf(z, 1e-30f);
        if (a.gate) o *= detector_sigmoid(a.gate[(int64_t)(sh / a.hq) * a.gate_stride + (sh % a.hq) * kHd + tid]);
        // with out_rotary R the head's rotary-pair order goes back to the exporter's
        // half-split column order (originalRotaryAxis), the columns the O projection's
        // axis remap reads (resident_quant.glsl:20,25)
        const int R = a.out_rotary;
        out[tid < R ? (tid & 1) * (R >> 1) + (tid >> 1) : tid] = o;
        if (tid == 0) {
            if (a.m_out) a.m_out[sh] = M;
            if (a.z_out) a.z_out[sh] = z;
            if (short_grid) raise_error(RTA_DEVERR_HITS);
        }
    }
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

// Tiles per chunk: 2, and 4 once the grid would cover 16384 tiles, so that the
// per-chunk records and prologue stay small next to the history they summarise.
static int attn_tiles(int nseq, int max_ctx) {
    const int64_t tiles = (int64_t)nseq * ((max_ctx + kTile - 1) / kTile);
    return tiles >= 16384 ? 4 : 2;
}

static int attn_lds_bytes(int hq, int hkv, int nblk, int fmt_v) {
    return AttnLds(hq, hkv, nblk, fmt_v == RTA_Q4_K ? Fmt<RTA_Q4_K>::kRow : Fmt<RTA_Q6_K>::kRow).total * 4;
}

template <int KF, int VF, int G, int KPW>
static hipError_t launch_chunk(const AttnArgs& a, int lds, hipStream_t s) {
    static int configured = 64 * 1024;   // raise the dynamic LDS limit when a launch needs more
    if (lds > configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_kernel<KF, VF, G, KPW>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        configured = lds;
    }
    hipLaunchKernelGGL((attn_chunk_kernel<KF, VF, G, KPW>), dim3(a.nchunk, a.nseq), dim3(256), lds, s, a);
    return hipGetLastError();
}

// Q4_K keys of at most 8 kv heads are scored on the matrix cores, with q operands
// prepared once per (sequence, kv head).
template <int G, int KPW, int NWV = 4>
static hipError_t launch_chunk_mma(const AttnArgs& a, hipStream_t s) {
    constexpr int lds = NWV * MmaWaveLds::total * 4;
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_mma_kernel<G, KPW, NWV>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL((attn_chunk_mma_kernel<G, KPW, NWV>), dim3(a.nwg), dim3(64 * NWV), lds, s, a);
    return hipGetLastError();
}

static int compute_units() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus = n;
    }
    return cus;
}

// Workgroups of the matrix-core kernels: per_cu per compute unit, all resident at once.
static int attn_mma_workgroups(int per_cu) {
    const int cus = compute_units();
    return per_cu * cus < kMaxWg ? per_cu * cus : kMaxWg;
}

// Workgroups per CU of attn_chunk_mma_kernel (Q4_K keys, Q6_K values): one 8-wave
// workgroup (one kv head per wave) when more than 4 kv heads share a superblock pair and
// the tile list cannot exceed one tile per CU (nseq x max_tiles <= CUs), else two 4-wave
// workgroups.  The tile plan (attn_qprep_kernel, full_middle_kernel) and the merge follow
// the same count.
static int mma_per_cu(int nseq, int64_t max_tiles, int hkv) {
    return (hkv > 4 && (int64_t)nseq * max_tiles <= compute_units()) ? 1 : 2;
}

// Q6_K keys with Q4_K values of at most 4 kv heads: scores and P V on the matrix cores.
template <int G>
static hipError_t launch_chunk_mma6(const AttnArgs& a, hipStream_t s) {
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_chunk_mma6_kernel<G>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kMma6LdsBytes);
        if (e != hipSuccess) return e;
        configured = true;
    }
    if (a.nseq > kWave) hipLaunchKernelGGL(attn_plan_kernel, dim3(1), dim3(kWave), 0, s, a);
    hipLaunchKernelGGL((attn_chunk_mma6_kernel<G>), dim3(a.nwg), dim3(256), kMma6LdsBytes, s, a);
    return hipGetLastError();
}

template <int KF, int VF, int G>
static hipError_t launch_chunk_k(const AttnArgs& a, int lds, hipStream_t s) {
    if constexpr (KF == RTA_Q6_K && VF == RTA_Q4_K) {
        if (a.hkv <= 4) return launch_chunk_mma6<G>(a, s);
    }
    if constexpr (KF == RTA_Q4_K) {
        if (a.hkv <= 8) {
            // (one more column of blocks builds the tile list of the matrix-core kernel)
            if (!a.prepared)
                hipLaunchKernelGGL((attn_qprep_kernel<G>), dim3(a.hkv + (a.plan ? 1 : 0), a.nseq), dim3(kWave), 0, s, a);
            if constexpr (VF == RTA_Q6_K) {   // scores and P V on the matrix cores
                if (a.hkv <= 4) return launch_chunk_mma<G, 1>(a, s);
                if (a.per_cu == 1) return launch_chunk_mma<G, 1, 8>(a, s);
                return launch_chunk_mma<G, 2>(a, s);
            }
            if (a.hkv <= 4) return launch_chunk<KF, VF, G, 1>(a, lds, s);
            return launch_chunk<KF, VF, G, 2>(a, lds, s);
        }
    }
    return launch_chunk<KF, VF, G, 0>(a, lds, s);
}

template <int KF, int VF>
static hipError_t launch_chunks(int G, const AttnArgs& a, int lds, hipStream_t s) {
    switch (G) {
    case 1: return launch_chunk_k<KF, VF, 1>(a, lds, s);
    case 2: return launch_chunk_k<KF, VF, 2>(a, lds, s);
    case 4: return launch_chunk_k<KF, VF, 4>(a, lds, s);
    default: return launch_chunk_k<KF, VF, 8>(a, lds, s);
    }
}

// ---- scratch of rta_decode_attention_noalloc ----------------------------------------
// The workspace of rta_decode_attention held in a file-scope device array, for callers
// that cannot allocate.  Each GPU the library runs on holds its own copy of the array
// (RTA_NOALLOC_SCRATCH_BYTES) until the process ends.  Every call on a GPU shares that
// GPU's copy, which keeps the last call's records: calls that overlap on one GPU race.
// Host code never uses the array's name as an address (on the host it is a stand-in):
// the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) uint8_t scratch[RTA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;

// Device address of the current device's scratch, looked up once per device with that
// device current.  RTA_OK or RTA_ERR_LAUNCH (no current device / the lookup failed).
static int scratch_address(void** out) {
    static std::mutex mu;
    static void* addr[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RTA_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RTA_ERR_LAUNCH;
        addr[dev] = p;
    }
    *out = addr[dev];
    return RTA_OK;
}


// ------------------------------------------------------------ dense receipts ----
// The standard backend's per-group attention records (resident_attention_dense.comp:
// 190-300 fusedAttention and storeHead, 118-126 the traversal count; layout
// attention_receipts.hpp:16-29, compact false).  Row r's history is its min(L, capacity)
// newest positions (L = ctx_len[r]); group g covers the ages [g block, g block + count)
// below its newest position, newest first.  Record (prefix(r) + g) hq + h, where
// prefix(r) sums the groups of the rows before r, holds hd + 8 + block / 32 words:
//   0 m, the group's maximum score q.k / sqrt(hd)      1 Z = sum exp(s - m)
//   2 count   3 exp evaluations   4 value runs   5 count
//   6 on head 0 the traversal count 2 + ceil(count / 16) that the reference's receipt
//     tracer reports for a group (two lens faces, one history ray per 16 positions), a
//     function of count alone; 0 on the other heads
//   7 flags: 3 (scores and values complete) | 4 (a weight was reused) | 8 (runs < count)
//   8 .. 8 + block / 32 the coverage bits (every position of the group is present)
//   then U_d = sum exp(s - m) v_d, d < hd.
// m, Z and U follow the reference's online order: tiles of four positions raise the
// running maximum (rescaling Z and U by exp(old - new) when it moves), a weight is reused
// when score and maximum repeat bit for bit, and consecutive bit-equal value vectors are
// summed as one run (weight sum times the vector), so words 3, 4 and 7 count the same
// events.  Block (head, group, row) of 256 threads: the four waves score the group's
// positions into LDS, then wave 0 runs the ordered pass with two axes per lane.
constexpr int kMaxReceiptBlock = 1024;
constexpr int kReceiptTile = 4;

__global__ void __launch_bounds__(256) attn_receipt_kernel(const float* __restrict__ q, int hq, int hkv,
                                                           const uint8_t* __restrict__ packets, int fmt_k, int fmt_v,
                                                           int64_t stride, int64_t v_offset,
                                                           const int64_t* __restrict__ slot_base,
                                                           const int32_t* __restrict__ ctx_len, int64_t capacity,
                                                           int64_t n_slots, int block, uint32_t* __restrict__ rec,
                                                           int64_t n_records) {
#pragma clang fp contract(off)
    __shared__ float s_q[kHd];
    __shared__ float s_score[kMaxReceiptBlock];
    __shared__ int64_t s_slot[kMaxReceiptBlock];
    __shared__ int s_bad;
    const int h = blockIdx.x, g = blockIdx.y, r = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t L = ctx_len[r];
    const int64_t active = L <= 0 ? 0 : (L < capacity ? L : capacity);
    if ((int64_t)g * block >= active) return;   // uniform: this row has fewer groups
    // a row with more groups than the grid holds (max_ctx below its length) is refused
    if (g == (int)gridDim.y - 1 && (int64_t)gridDim.y * block < active) {
        if (tid == 0) raise_error(RTA_DEVERR_HITS);
        return;
    }
    int64_t prefix = 0;
    for (int rr = 0; rr < r; ++rr) {
        const int64_t l = ctx_len[rr], a = l <= 0 ? 0 : (l < capacity ? l : capacity);
        prefix += (a + block - 1) / block;
    }
    const int64_t record = (prefix + g) * hq + h;
    if (record >= n_records) {
        if (tid == 0) raise_error(RTA_DEVERR_HITS);
        return;
    }
    const int count = (int)(active - (int64_t)g * block < block ? active - (int64_t)g * block : block);
    const int kv = h / (hq / hkv);
    if (tid == 0) s_bad = 0;
    if (tid < kHd) s_q[tid] = q[((int64_t)r * hq + h) * kHd + tid];
    __syncthreads();
    for (int j = tid; j < count; j += 256) {
        const int64_t p = L - 1 - ((int64_t)g * block + j);
        const int64_t slot = slot_base[r] + p % capacity;
        const bool bad = slot < 0 || slot >= n_slots;
        if (bad) s_bad = 1;
        s_slot[j] = bad ? 0 : slot;
    }
    __syncthreads();
    if (s_bad) {
        if (tid == 0) raise_error(RTA_DEVERR_HITS);
        return;
    }
    // Scores: a wave per position, lane holds axes lane and lane + 64.
    const float qa = s_q[lane], qb = s_q[lane + 64];
    const bool q_ok = isfinite(qa) && isfinite(qb);
    bool finite = q_ok;
    const int64_t kbase = (int64_t)kv * kHd;
    for (int j = wave; j < count; j += 4) {
        const uint8_t* kf = packets + s_slot[j] * stride;
        const float ka = dequant_value(fmt_k, kf, kbase + lane), kb = dequant_value(fmt_k, kf, kbase + lane + 64);
        finite &= isfinite(ka) && isfinite(kb);
        const float pa = qa * ka, pb = qb * kb;
        float t = pa + pb;
        for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, kWave);
        const float score = t / sqrtf((float)kHd);
        finite &= isfinite(score);
        if (lane == 0) s_score[j] = score;
    }
    if (!finite) raise_error(RTA_DEVERR_DETECTOR);
    __syncthreads();
    if (wave != 0) return;
    float maximum = -INFINITY, reference = 0.0f, pending_w = 0.0f, prev_w = 0.0f;
    float sig_a = 0.0f, sig_b = 0.0f, pv_a = 0.0f, pv_b = 0.0f;
    uint32_t prev_score = 0u, prev_max = 0u, exps = 0u, runs = 0u;
    bool pending = false, have_prev = false, reused = false, vfinite = true;
    for (int t0 = 0; t0 < count; t0 += kReceiptTile) {
        const int n = count - t0 < kReceiptTile ? count - t0 : kReceiptTile;
        float local = -INFINITY;
        for (int j = 0; j < n; ++j) local = fmaxf(local, s_score[t0 + j]);
        const float next = fmaxf(maximum, local);
        float scale = 0.0f;
        if (reference > 0.0f) {
            if (__float_as_uint(next) == __float_as_uint(maximum)) {
                scale = 1.0f;
            } else {
                scale = expf(maximum - next);
                ++exps;
            }
        }
        reference *= scale;
        pending_w *= scale;
        sig_a *= scale;
        sig_b *= scale;
        maximum = next;
        for (int j = 0; j < n; ++j) {
            const float score = s_score[t0 + j];
            float w;
            if (have_prev && __float_as_uint(score) == prev_score && __float_as_uint(maximum) == prev_max) {
                w = prev_w;
                reused = true;
            } else {
                w = expf(score - maximum);
                ++exps;
            }
            prev_score = __float_as_uint(score);
            prev_max = __float_as_uint(maximum);
            prev_w = w;
            have_prev = true;
            reference += w;
            const uint8_t* vf = packets + s_slot[t0 + j] * stride + v_offset;
            const float va = dequant_value(fmt_v, vf, kbase + lane), vb = dequant_value(fmt_v, vf, kbase + lane + 64);
            vfinite &= isfinite(va) && isfinite(vb);
            const bool same = pending && __float_as_uint(va) == __float_as_uint(pv_a) &&
                              __float_as_uint(vb) == __float_as_uint(pv_b);
            if (__all(same)) {
                pending_w += w;
            } else {
                if (pending) {
                    const float ca = pending_w * pv_a, cb = pending_w * pv_b;
                    sig_a += ca;
                    sig_b += cb;
                    ++runs;
                }
                pv_a = va;
                pv_b = vb;
                pending_w = w;
                pending = true;
            }
        }
    }
    if (pending) {
        const float ca = pending_w * pv_a, cb = pending_w * pv_b;
        sig_a += ca;
        sig_b += cb;
        ++runs;
    }
    if (!vfinite || !isfinite(reference) || !(reference > 0.0f) || !isfinite(maximum) || !isfinite(sig_a) ||
        !isfinite(sig_b))
        raise_error(RTA_DEVERR_DETECTOR);
    uint32_t* out = rec + record * (int64_t)(kHd + 8 + block / 32);
    const int cov = block / 32;
    out[8 + cov + lane] = __float_as_uint(sig_a);
    out[8 + cov + lane + 64] = __float_as_uint(sig_b);
    for (int w = lane; w < cov; w += 64) {
        const int first = 32 * w, nb = first < count ? (count - first < 32 ? count - first : 32) : 0;
        out[8 + w] = nb == 32 ? 0xFFFFFFFFu : nb == 0 ? 0u : (1u << nb) - 1u;
    }
    if (lane == 0) {
        out[0] = __float_as_uint(maximum);
        out[1] = __float_as_uint(reference);
        out[2] = (uint32_t)count;
        out[3] = exps;
        out[4] = runs;
        out[5] = (uint32_t)count;
        out[6] = h == 0 ? 2u + (uint32_t)(count + 15) / 16u : 0u;
        out[7] = 3u | (reused ? 4u : 0u) | (runs < (uint32_t)count ? 8u : 0u);
    }
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

// Chunk records [nseq][nchunk][hq][kRec] floats, then the matrix-core q operands
// [nseq][hkv][6][64] 16-byte words.
static size_t attn_record_bytes(int nseq, int hq, int max_ctx) {
    // room for one record per tile (the chunk grid needs one per chunk, the tile-list
    // split at most one per tile of the sequence)
    const int64_t tiles = ((int64_t)max_ctx + kTile - 1) / kTile;
    return (size_t)nseq * (size_t)tiles * (size_t)hq * kRec * sizeof(float);
}

size_t rta_decode_attention_workspace_bytes(int nseq, int hq, int hkv, int hd, int max_ctx) {
    if (nseq <= 0 || hq <= 0 || hkv <= 0 || hd != kHd || max_ctx <= 0 || hq % hkv) return 0;
    return attn_record_bytes(nseq, hq, max_ctx) + (size_t)nseq * hkv * 6 * kWave * sizeof(uint4) +
           (((size_t)nseq + 1 + kMaxWg) * sizeof(int32_t) + 15) / 16 * 16;
}

int64_t rta_attention_receipt_records(const int32_t* ctx_len_host, int rows, int hq, int64_t capacity, int block) {
    if (!ctx_len_host || rows <= 0 || hq <= 0 || capacity <= 0 || block <= 0) return -1;
    int64_t n = 0;
    for (int r = 0; r < rows; ++r) {
        const int64_t L = ctx_len_host[r], active = L < capacity ? L : capacity;
        if (active > 0) n += (active + block - 1) / block;
    }
    return n * hq;
}

int rta_attention_receipts(const float* q, int rows, int hq, int hkv, int hd, const void* packets, int fmt_k,
                           int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                           int64_t n_slots, int max_ctx, int block, uint32_t* receipts, int64_t n_records,
                           rta_stream_t stream) {
    if (!q || !packets || !slot_base || !ctx_len || !receipts) return RTA_ERR_NULL;
    if (rows <= 0 || hq <= 0 || hkv <= 0 || hq % hkv || capacity <= 0 || n_slots <= 0 || max_ctx <= 0 ||
        n_records <= 0)
        return RTA_ERR_SHAPE;
    if ((fmt_k != RTA_Q4_K && fmt_k != RTA_Q6_K) || (fmt_v != RTA_Q4_K && fmt_v != RTA_Q6_K) ||
        (fmt_k == RTA_Q6_K && fmt_v == RTA_Q6_K))
        return RTA_ERR_FORMAT;
    if (hd != kHd || block < 32 || block % 32 || block > kMaxReceiptBlock) return RTA_ERR_RANGE;
    if (!host::aligned(q, 4) || !host::aligned(slot_base, 8) || !host::aligned(ctx_len, 4) ||
        !host::aligned(receipts, 4))
        return RTA_ERR_ALIGN;
    const int64_t lim = (int64_t)max_ctx < capacity ? max_ctx : capacity;
    const int64_t groups = (lim + block - 1) / block;
    if (groups > 65535 || rows > 65535) return RTA_ERR_RANGE;
    const int nkv2 = (hkv * kHd + 255) / 256;
    const int64_t stride = host::history_bytes(hkv * kHd);
    const int64_t v_offset = (int64_t)nkv2 * (fmt_k == RTA_Q4_K ? 144 : 210);
    hipLaunchKernelGGL(attn_receipt_kernel, dim3(hq, (unsigned)groups, rows), dim3(256), 0, (hipStream_t)stream, q,
                       hq, hkv, static_cast<const uint8_t*>(packets), fmt_k, fmt_v, stride, v_offset, slot_base,
                       ctx_len, capacity, n_slots, block, receipts, n_records);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_decode_attention(const float* q, int nseq, int hq, int hkv, int hd, const void* packets, int fmt_k, int fmt_v,
                         const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity, int64_t n_slots,
                         int max_ctx, const float* gate, float* out, float* m_out, float* z_out, void* workspace,
                         size_t workspace_bytes, rta_stream_t stream) {
    return decode_attention_gate_stride(q, nseq, hq, hkv, hd, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity,
                                        n_slots, max_ctx, gate, (int64_t)hq * hd, out, m_out, z_out, workspace,
                                        workspace_bytes, stream);
}

}  // extern "C"

namespace rta {

int attention_shape_check(int hq, int hkv, int hd, int fmt_k, int fmt_v) {
    if (hq <= 0 || hkv <= 0 || hd <= 0 || hq % hkv) return RTA_ERR_SHAPE;
    if ((fmt_k != RTA_Q4_K && fmt_k != RTA_Q6_K) || (fmt_v != RTA_Q4_K && fmt_v != RTA_Q6_K)) return RTA_ERR_FORMAT;
    // a packet holds 354 bytes per 256 values (resident_dimensions.hpp:10): one Q4_K and one
    // Q6_K field, or two Q4_K fields; two Q6_K fields would overrun it
    if (fmt_k == RTA_Q6_K && fmt_v == RTA_Q6_K) return RTA_ERR_FORMAT;
    const int G = hq / hkv;
    if (hd != kHd || (G != 1 && G != 2 && G != 4 && G != 8)) return RTA_ERR_RANGE;
    // phase B spreads every kv head over 128 / (8 or 16) threads of one 256-thread workgroup
    if (hkv * (G == 8 ? 16 : 8) > 256) return RTA_ERR_RANGE;
    const int nblk = (hkv * kHd + 255) / 256;
    if (attn_lds_bytes(hq, hkv, nblk, fmt_v) > kMaxLds) return RTA_ERR_RANGE;
    return RTA_OK;
}

int decode_attention_gate_stride(const float* q, int nseq, int hq, int hkv, int hd, const void* packets, int fmt_k,
                                 int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                                 int64_t n_slots, int max_ctx, const float* gate, int64_t gate_stride, float* out,
                                 float* m_out, float* z_out, void* workspace, size_t workspace_bytes,
                                 rta_stream_t stream, int out_rotary, bool prepared) {
    if (!q || !packets || !slot_base || !ctx_len || !out) return RTA_ERR_NULL;   // m_out, z_out optional
    if (nseq <= 0 || capacity <= 0 || max_ctx <= 0 || n_slots <= 0) return RTA_ERR_SHAPE;
    const int shape_rc = attention_shape_check(hq, hkv, hd, fmt_k, fmt_v);
    if (shape_rc) return shape_rc;
    const int G = hq / hkv;
    const int nblk = (hkv * kHd + 255) / 256;
    const int lds = attn_lds_bytes(hq, hkv, nblk, fmt_v);
    if (!host::aligned(q, 4) || !host::aligned(packets, 4) || !host::aligned(slot_base, 8) ||
        !host::aligned(ctx_len, 4) || !host::aligned(out, 4) || (gate && !host::aligned(gate, 4)))
        return RTA_ERR_ALIGN;
    if (gate && gate_stride < (int64_t)hq * hd) return RTA_ERR_SHAPE;
    const size_t need = rta_decode_attention_workspace_bytes(nseq, hq, hkv, hd, max_ctx);
    if (!workspace || workspace_bytes < need || !host::aligned(workspace, 16)) return RTA_ERR_WORKSPACE;
    AttnArgs a{};
    a.q = q;
    a.packets = static_cast<const uint8_t*>(packets);
    a.slot_base = slot_base;
    a.ctx_len = ctx_len;
    a.gate = gate;
    a.gate_stride = gate_stride;
    if (out_rotary < 0 || out_rotary > hd || out_rotary % 2) return RTA_ERR_RANGE;
    a.out_rotary = out_rotary;
    a.prepared = prepared;
    a.out = out;
    a.m_out = m_out;
    a.z_out = z_out;
    a.ws = static_cast<float*>(workspace);
    a.qop = reinterpret_cast<uint4*>(static_cast<uint8_t*>(workspace) + attn_record_bytes(nseq, hq, max_ctx));
    a.capacity = capacity;
    a.n_slots = n_slots;
    const int kvw = hkv * kHd;
    a.stride = host::history_bytes(kvw);
    a.v_offset = (int64_t)nblk * (fmt_k == RTA_Q4_K ? 144 : 210);
    a.nseq = nseq;
    a.hq = hq;
    a.hkv = hkv;
    a.nt = attn_tiles(nseq, max_ctx);
    a.nchunk = (int)((max_ctx + a.nt * kTile - 1) / (a.nt * kTile));
    a.nblk = nblk;
    a.max_tiles = ((int64_t)max_ctx + kTile - 1) / kTile;
    if ((fmt_k == RTA_Q4_K && fmt_v == RTA_Q6_K && hkv <= 8) ||
        (fmt_k == RTA_Q6_K && fmt_v == RTA_Q4_K && hkv <= 4)) {   // the matrix-core kernels' tile-list split
        a.plan = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(a.qop) + (size_t)nseq * hkv * 6 * kWave * sizeof(uint4));
        a.per_cu = fmt_k == RTA_Q6_K ? kMma6PerCu : mma_per_cu(nseq, a.max_tiles, hkv);
        a.nwg = attn_mma_workgroups(a.per_cu);
        a.rstride = a.max_tiles;
    }
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    if (fmt_k == RTA_Q4_K && fmt_v == RTA_Q6_K) e = launch_chunks<RTA_Q4_K, RTA_Q6_K>(G, a, lds, s);
    else if (fmt_k == RTA_Q6_K && fmt_v == RTA_Q4_K) e = launch_chunks<RTA_Q6_K, RTA_Q4_K>(G, a, lds, s);
    else e = launch_chunks<RTA_Q4_K, RTA_Q4_K>(G, a, lds, s);
    if (e != hipSuccess) return RTA_ERR_LAUNCH;
    if (nseq <= 16) hipLaunchKernelGGL((attn_merge_kernel<16>), dim3(nseq * hq), dim3(512), 0, s, a);
    else hipLaunchKernelGGL((attn_merge_kernel<8>), dim3(nseq * hq), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int full_layer_middle(const float* proj, int64_t slab_stride, int row_stride, int nslab, int batch, int hq, int hkv,
                      const float* q_norm, const float* k_norm, float eps, const int64_t* positions, int rotary,
                      double theta, float* q_out, float* gate_out, int64_t gate_stride, int fmt_k, int fmt_v,
                      const int64_t* slots, int64_t n_slots, void* packets, const int32_t* ctx_len, int64_t capacity,
                      int max_ctx, void* attn_ws, float* kv_out, hipStream_t s) {
    if (!proj || !positions || !q_out || !slots || !packets || !ctx_len || !attn_ws) return RTA_ERR_NULL;
    if (batch <= 0 || hq <= 0 || hkv <= 0 || hq % hkv || row_stride < (2 * hq + 2 * hkv) * kHd - (gate_out ? 0 : hq * kHd))
        return RTA_ERR_SHAPE;
    if (nslab <= 0 || nslab > 16 || rotary < 0 || rotary > kHd || rotary % 2) return RTA_ERR_RANGE;
    if ((fmt_k != RTA_Q4_K && fmt_k != RTA_Q6_K) || (fmt_v != RTA_Q4_K && fmt_v != RTA_Q6_K) ||
        (fmt_k == RTA_Q6_K && fmt_v == RTA_Q6_K))
        return RTA_ERR_FORMAT;
    const int G = hq / hkv;
    MiddleArgs p{};
    p.proj = proj;
    p.slab_stride = slab_stride;
    p.row_stride = row_stride;
    p.nslab = nslab;
    p.hq = hq;
    p.hkv = hkv;
    p.G = G;
    p.q_norm = q_norm;
    p.k_norm = k_norm;
    p.eps = eps;
    p.positions = positions;
    p.rotary = rotary;
    p.theta = theta;
    p.q_out = q_out;
    p.gate_out = gate_out;
    p.gate_stride = gate_stride;
    p.fmt_k = fmt_k;
    p.fmt_v = fmt_v;
    p.slot = slots;
    p.n_slots = n_slots;
    p.stride = host::history_bytes(hkv * kHd);
    p.nkv2 = (hkv * kHd + 255) / 256;
    p.v_offset = (int64_t)p.nkv2 * (fmt_k == RTA_Q4_K ? 144 : 210);
    p.packets = static_cast<uint8_t*>(packets);
    p.kv_out = kv_out;
    p.nqb = (hq + 3) / 4;
    // the attention kernels for Q4_K keys of at most 8 kv heads read matrix-core q operands
    // (and, with Q6_K values, a tile plan) that rta_decode_attention keeps in its
    // workspace: written here instead
    const bool qops = fmt_k == RTA_Q4_K && hkv <= 8 && (G == 1 || G == 2 || G == 4 || G == 8);
    if (qops) p.qop = reinterpret_cast<uint4*>(static_cast<uint8_t*>(attn_ws) + attn_record_bytes(batch, hq, max_ctx));
    if (qops && fmt_v == RTA_Q6_K) {
        AttnArgs& a = p.plan;
        a.nseq = batch;
        a.ctx_len = ctx_len;
        a.capacity = capacity;
        a.max_tiles = ((int64_t)max_ctx + kTile - 1) / kTile;
        a.per_cu = mma_per_cu(batch, a.max_tiles, hkv);
        a.nwg = attn_mma_workgroups(a.per_cu);
        a.plan = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(p.qop) +
                                            (size_t)batch * hkv * 6 * kWave * sizeof(uint4));
    }
    const dim3 g(p.nqb + p.nkv2 + (p.plan.plan ? 1 : 0), batch), blk(256);
    if (nslab == 1) hipLaunchKernelGGL((full_middle_kernel<1>), g, blk, 0, s, p);
    else if (nslab == 2) hipLaunchKernelGGL((full_middle_kernel<2>), g, blk, 0, s, p);
    else if (nslab <= 4) hipLaunchKernelGGL((full_middle_kernel<4>), g, blk, 0, s, p);
    else if (nslab <= 8) hipLaunchKernelGGL((full_middle_kernel<8>), g, blk, 0, s, p);
    else hipLaunchKernelGGL((full_middle_kernel<16>), g, blk, 0, s, p);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

}  // namespace rta

extern "C" {

int rta_decode_attention_noalloc(const float* q, int nseq, int hq, int hkv, int hd, const void* packets, int fmt_k,
                                 int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                                 int64_t n_slots, int max_ctx, const float* gate, float* out, float* m_out,
                                 float* z_out, rta_stream_t stream) {
    const size_t need = rta_decode_attention_workspace_bytes(nseq, hq, hkv, hd, max_ctx);
    // need == 0: an invalid shape, reported by rta_decode_attention's own checks
    if (need > RTA_NOALLOC_SCRATCH_BYTES) return RTA_ERR_SCRATCH;
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc) return rc;
    return rta_decode_attention(q, nseq, hq, hkv, hd, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity, n_slots,
                                max_ctx, gate, out, m_out, z_out, ws, RTA_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
