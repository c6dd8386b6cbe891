// rta_pack.hpp -- the history packer's quantisation of one superblock (256 values) of
// a key field and of a value field, shared by rta_pack_history and by the decode
// step's full-layer middle kernel, so both write the same bytes by construction.
//
// op 34 (resident_history_quant.glsl:9-41), every step in the reference's fp32 order
// (contraction off, IEEE division, round-half-even codes, fp16 block scales):
//   Q4_K field: 32-value groups; lo and hi start at 0 (:14), so a group's span is
//               (max(0, max x) - min(0, min x)) / 15 and its minimum -min(0, min x);
//               d = fp16(max span / 63), dmin = fp16(max minimum / 63), 6-bit codes
//   Q6_K field: 16-value groups, max|x| / 31, d = fp16(max / 127), 8-bit codes
#pragma once
#include "rta_common.hpp"

namespace rta {

// GLSL min / max: x unless y is strictly smaller / larger.  They fix the sign of zero
// where the packer compares +0 with -0 (the minimum -min(0, x) of an all-zero group is
// -0), which the fp16 block minimum keeps.
__device__ __forceinline__ float glsl_min(float x, float y) { return y < x ? y : x; }
__device__ __forceinline__ float glsl_max(float x, float y) { return x < y ? y : x; }

// LDS scratch of one field superblock.
struct PackScratch {
    float gscale[16], gmin[16], bd, bdm;
    uint32_t sc[16], mn[16];
};

// 1. group statistics (:11-17): thread t < groups
__device__ __forceinline__ void pack_stats(const float* xs, bool q4, PackScratch& st, int t) {
#pragma clang fp contract(off)
    const int ng = q4 ? 8 : 16, width = q4 ? 32 : 16;
    if (t < ng) {
        float lo = 0.0f, hi = 0.0f;
        for (int i = 0; i < width; ++i) {
            const float v = xs[t * width + i];
            if (q4) {
                lo = glsl_min(lo, v);
                hi = glsl_max(hi, v);
            } else {
                hi = glsl_max(hi, fabsf(v));
            }
        }
        st.gscale[t] = q4 ? (hi - lo) / 15.0f : hi / 31.0f;
        st.gmin[t] = q4 ? -lo : 0.0f;
    }
}

// 2. block scales rounded to fp16 and their header bytes (:18-24): one thread
__device__ __forceinline__ void pack_scales(bool q4, PackScratch& st, uint8_t* out) {
#pragma clang fp contract(off)
    const int ng = q4 ? 8 : 16;
    float maxD = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < ng; ++g) {
        maxD = glsl_max(maxD, st.gscale[g]);
        maxMin = glsl_max(maxMin, st.gmin[g]);
    }
    const _Float16 hd16 = (_Float16)(maxD / (q4 ? 63.0f : 127.0f));
    st.bd = (float)hd16;
    const uint16_t hb = __builtin_bit_cast(uint16_t, hd16);
    if (q4) {
        const _Float16 hm16 = (_Float16)(maxMin / 63.0f);
        st.bdm = (float)hm16;
        const uint16_t hm = __builtin_bit_cast(uint16_t, hm16);
        out[0] = hb & 255;
        out[1] = hb >> 8;
        out[2] = hm & 255;
        out[3] = hm >> 8;
    } else {
        out[208] = hb & 255;
        out[209] = hb >> 8;
    }
}

// 3. group scale / minimum codes (:25-30): thread t < groups
__device__ __forceinline__ void pack_codes(bool q4, PackScratch& st, uint8_t* out, int t) {
#pragma clang fp contract(off)
    const int ng = q4 ? 8 : 16;
    if (t < ng) {
        st.sc[t] = (uint32_t)fminf(fmaxf(rintf(st.gscale[t] / fmaxf(st.bd, 1e-30f)), 0.0f), q4 ? 63.0f : 127.0f);
        if (q4) st.mn[t] = (uint32_t)fminf(fmaxf(rintf(st.gmin[t] / fmaxf(st.bdm, 1e-30f)), 0.0f), 63.0f);
        else out[192 + t] = (uint8_t)st.sc[t];
    }
}

// 4. the packed 6-bit Q4_K scales (:31-33) and the quantised values (:34-38), one
// output byte per thread t < 192
__device__ __forceinline__ void pack_values(const float* xs, bool q4, const PackScratch& st, uint8_t* out, int t) {
#pragma clang fp contract(off)
    if (q4 && t < 4) {
        out[4 + t] = (uint8_t)(st.sc[t] | ((st.sc[t + 4] >> 4) << 6));
        out[8 + t] = (uint8_t)(st.mn[t] | ((st.mn[t + 4] >> 4) << 6));
        out[12 + t] = (uint8_t)((st.sc[t + 4] & 15u) | ((st.mn[t + 4] & 15u) << 4));
    }
    auto q4code = [&](int i) {
        const int g = i >> 5;
        const float num = xs[i] + st.bdm * (float)st.mn[g];
        const float den = fmaxf(st.bd * (float)st.sc[g], 1e-30f);
        return (uint32_t)fminf(fmaxf(rintf(num / den), 0.0f), 15.0f);
    };
    auto q6code = [&](int i) {
        const int g = i >> 4;
        const float den = fmaxf(st.bd * (float)st.sc[g], 1e-30f);
        return (uint32_t)((int)fminf(fmaxf(rintf(xs[i] / den), -32.0f), 31.0f) + 32);
    };
    if (q4) {
        if (t < 128) {   // qs byte t: value 64 (t/32) + t%32 (low nibble) and +32 (high)
            const int i = 64 * (t >> 5) + (t & 31);
            out[16 + t] = (uint8_t)(q4code(i) | (q4code(i + 32) << 4));
        }
    } else if (t < 128) {   // ql byte: value 128 (t/64) + t%64 (low) and +64 (high)
        const int i = 128 * (t >> 6) + (t & 63);
        out[t] = (uint8_t)((q6code(i) & 15u) | ((q6code(i + 64) & 15u) << 4));
    } else if (t < 192) {   // qh byte: values 128 part + l + 32 k, two bits each
        const int jj = t - 128, i = 128 * (jj >> 5) + (jj & 31);
        out[t] = (uint8_t)(((q6code(i) >> 4) & 3u) | (((q6code(i + 32) >> 4) & 3u) << 2) |
                           (((q6code(i + 64) >> 4) & 3u) << 4) | (((q6code(i + 96) >> 4) & 3u) << 6));
    }
}

// One superblock of each field: xs[0] the key values, xs[1] the value values (256
// each, zero past the row), q4[f] whether field f is Q4_K (else Q6_K); out[f] receives
// its 144 / 210 bytes.  Every one of a block's 256 threads calls it (it holds block
// barriers); xs must be visible to all of them (a barrier after it was written).
__device__ __forceinline__ void pack_superblock_pair(const float (*xs)[256], const bool* q4, PackScratch* st,
                                                     uint8_t (*out)[212], int tid) {
    pack_stats(xs[0], q4[0], st[0], tid);
    if (tid >= 64 && tid < 128) pack_stats(xs[1], q4[1], st[1], tid - 64);
    __syncthreads();
    if (tid == 0) pack_scales(q4[0], st[0], out[0]);
    if (tid == 64) pack_scales(q4[1], st[1], out[1]);
    __syncthreads();
    pack_codes(q4[0], st[0], out[0], tid);
    if (tid >= 64 && tid < 128) pack_codes(q4[1], st[1], out[1], tid - 64);
    __syncthreads();
    pack_values(xs[0], q4[0], st[0], out[0], tid);
    pack_values(xs[1], q4[1], st[1], out[1], tid);
    __syncthreads();
}

}  // namespace rta
