// rta_common.hpp -- device helpers shared by the gfx950 kernels.
//
// Quantised formats follow the reference decoder byte for byte
// (ray_tracing/native/shaders/resident_quant.glsl:6-20):
//   Q4_K superblock (144 B): d f16 | dmin f16 | 12 scale bytes | 128 nibble bytes
//   Q6_K superblock (210 B): 128 ql | 64 qh | 16 int8 scales | d f16
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/rta.h"

namespace rta {

constexpr int kWave = 64;

// Sticky device error word; bits as RTA_DEVERR_* (the reference's control[3]).
extern __device__ uint32_t g_error_word;

__device__ __forceinline__ void raise_error(uint32_t bit) { atomicOr(&g_error_word, bit); }

// IEEE binary16 -> binary32 for the low / high half of a dword (exact).
__device__ __forceinline__ float half_lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Reinterprets a dword whose halves hold small integer codes c (bits 0..9) as two
// binary16 subnormals c * 2^-24.  Converting such a half to fp32 is exact, so
// fmaf((float)h.x, x, acc) accumulates c * x * 2^-24 with one v_fma_mix_f32.
__device__ __forceinline__ half2_t as_codes(uint32_t w) { return __builtin_bit_cast(half2_t, w); }

// (hi:lo) >> (8 * shift) -- extracts a dword that starts `shift` bytes into lo.
__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// Butterfly sum over lanes whose index differs only in the bits below `width`
// (a power of two <= 64).  Every lane of the group ends with the group sum.
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}



template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// The gfx950 row swaps with v as both operands (v_permlane16_swap / v_permlane32_swap):
// every lane gets the value of its lane position in the even and the odd 16-lane row of
// its row pair, or in the lower and the upper 32-lane half.  No LDS round trip.
__device__ __forceinline__ void rows16_pair(float v, float& even, float& odd) {
    const int b = __builtin_bit_cast(int, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    even = __builtin_bit_cast(float, (int)r[0]);
    odd = __builtin_bit_cast(float, (int)r[1]);
}
__device__ __forceinline__ void halves32(float v, float& lo, float& hi) {
    const int b = __builtin_bit_cast(int, v);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    lo = __builtin_bit_cast(float, (int)r[0]);
    hi = __builtin_bit_cast(float, (int)r[1]);
}
// v + the value of lane ^ 16 (^ 32), as (even row + odd row) (lower + upper half) in
// every lane: the sum a butterfly step forms, since addition commutes
__device__ __forceinline__ float add_xor16(float v) {
    float e, o;
    rows16_pair(v, e, o);
    return e + o;
}
__device__ __forceinline__ float add_xor32(float v) {
    float l, h;
    halves32(v, l, h);
    return l + h;
}
__device__ __forceinline__ float max_xor16(float v) {
    float e, o;
    rows16_pair(v, e, o);
    return fmaxf(e, o);
}
__device__ __forceinline__ float max_xor32(float v) {
    float l, h;
    halves32(v, l, h);
    return fmaxf(l, h);
}

// Sum / max over the 64 lanes of a wave, every lane getting the same result: DPP
// steps inside each 16-lane row (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror), then the two row swaps.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    return add_xor32(add_xor16(v));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return max_xor32(max_xor16(v));
}

// Integer minimum over the 64 lanes, every lane getting it (the same DPP steps and row
// swaps as wave_max_dpp).
__device__ __forceinline__ int wave_min_int(int v) {
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true));
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = min((int)r[0], (int)r[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return min((int)q[0], (int)q[1]);
}

// Max over the lanes whose index differs only in the bits below `width` (a power of two
// <= 64); every lane of the group ends with the group maximum (exact in any order).
__device__ __forceinline__ float group_max(float v, int width) {
    if (width >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
    if (width >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
    if (width >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
    if (width >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
    if (width >= 32) v = max_xor16(v);
    if (width >= 64) v = max_xor32(v);
    return v;
}

// Q4_K 6-bit scale/min codes of group g (0..7) from the scale dwords
// s0 = bytes 4..7, s1 = bytes 8..11, s2 = bytes 12..15 of the superblock
// (resident_quant.glsl:11-12, q4ScaleMin :39-43).
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int g,
                                              uint32_t& sc, uint32_t& m) {
    const uint32_t sh = 8u * (uint32_t)(g & 3);
    const uint32_t a = (s0 >> sh) & 255u, b = (s1 >> sh) & 255u;
    if (g < 4) {
        sc = a & 63u;
        m = b & 63u;
    } else {
        const uint32_t mixed = (s2 >> sh) & 255u;
        sc = (mixed & 15u) | ((a >> 6) << 4);
        m = (mixed >> 4) | ((b >> 6) << 4);
    }
}

// Scale and minimum of Q4_K group g (0..7, may differ between lanes), without a
// branch: both forms are computed and one is kept by a bit mask (a lane-dependent
// ternary compiles to two exec-masked paths).
__device__ __forceinline__ void q4k_scale_min_lane(uint32_t s0, uint32_t s1, uint32_t s2, int g, uint32_t& sc,
                                                   uint32_t& m) {
    const uint32_t sh = 8u * (uint32_t)(g & 3);
    const uint32_t a = s0 >> sh, b = s1 >> sh, mixed = s2 >> sh;
    const uint32_t sc_lo = a & 63u, m_lo = b & 63u;
    const uint32_t sc_hi = (mixed & 15u) | ((a >> 2) & 0x30u), m_hi = ((mixed >> 4) & 15u) | ((b >> 2) & 0x30u);
    const uint32_t keep_lo = g < 4 ? 0xFFFFFFFFu : 0u;
    sc = (sc_lo & keep_lo) | (sc_hi & ~keep_lo);
    m = (m_lo & keep_lo) | (m_hi & ~keep_lo);
}

// ---- matrix-core operand helpers (v_mfma_f32_16x16x32_f16) ----

// Exponent e of a block maximum mx = f 2^e (f in [0.5, 1)) for the power-of-two operand
// scale 2^(14 - e) that puts the block's largest value in [2^13, 2^14): 0 for a zero or
// non-finite maximum, and never below -110, so that the scale (<= 2^124) and its inverse
// (>= 2^-124) stay finite normal fp32 numbers.  A block whose maximum is below 2^-111
// (fp32 subnormals among them) is scaled by 2^124 only; it loses relative precision,
// never finiteness.
__device__ __forceinline__ int operand_exponent(float mx) {
    int e = 0;
    if (mx > 0.0f && isfinite(mx)) (void)frexpf(mx, &e);
    return e < -110 ? -110 : e;
}

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h2v_t __attribute__((ext_vector_type(2)));

// Two binary16 products in one v_pk_mul_f16 (a code pair times a duplicated scale).
__device__ __forceinline__ uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v_t, a) * __builtin_bit_cast(h2v_t, b));
}

// (f16(v), f16(v)) for a value v exactly representable in binary16
__device__ __forceinline__ uint32_t h2dup(float v) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)v);
    return h | (h << 16);
}

// A deferred RMSNorm for the readouts: x was written as h * w without the row factor;
// the readout multiplies row r's result by 1 / sqrt((p.x + p.y + p.z + p.w) / width + eps),
// p = part[r] the row's four column-chunk sums of squares (16-byte aligned, unused
// chunks zero).  part == nullptr: no factor.
struct RowNorm {
    const float4* part = nullptr;
    float width = 0.0f;
    float eps = 0.0f;
};

__device__ __forceinline__ float row_norm_factor(const RowNorm& rn, float4 p) {
    return 1.0f / sqrtf((((p.x + p.y) + p.z) + p.w) / rn.width + rn.eps);
}

// Value i of a GGUF-encoded array, with the reference decoder's fp32 op order
// (resident_quant.glsl:6-20); contraction is disabled so that (d*sc)*q - dmin*m is
// rounded exactly as the reference rounds it.
__device__ __forceinline__ float dequant_value(int fmt, const uint8_t* __restrict__ src, int64_t i) {
#pragma clang fp contract(off)
    if (fmt == RTA_F32) return reinterpret_cast<const float*>(src)[i];
    if (fmt == RTA_F16) return (float)reinterpret_cast<const _Float16*>(src)[i];
    if (fmt == RTA_BF16) return __builtin_bit_cast(float, (uint32_t)reinterpret_cast<const uint16_t*>(src)[i] << 16);
    if (fmt == RTA_Q4_K) {
        // A Q4_K field that follows a Q6_K field in a history packet starts 2 bytes past
        // a word boundary (210-byte blocks), so the header is read in 16-bit halves: a
        // 32-bit read there, when the address is wave-uniform, may be served by a scalar
        // load, which drops the low address bits.
        const uint8_t* b = src + (i >> 8) * 144;
        const uint16_t* hw = reinterpret_cast<const uint16_t*>(b);
        const int idx = (int)(i & 255), g = idx >> 5;
        const float d = (float)__builtin_bit_cast(_Float16, hw[0]);
        const float dmin = (float)__builtin_bit_cast(_Float16, hw[1]);
        uint32_t sc, m;
        q4k_scale_min(hw[2] | (uint32_t)hw[3] << 16, hw[4] | (uint32_t)hw[5] << 16, hw[6] | (uint32_t)hw[7] << 16, g,
                      sc, m);
        const uint32_t q = (b[16 + (idx >> 6) * 32 + (idx & 31)] >> (((idx & 63) >> 5) * 4)) & 15u;
        const float ds = d * (float)sc;
        const float dq = ds * (float)q;
        const float dm = dmin * (float)m;
        return dq - dm;
    }
    const uint8_t* b = src + (i >> 8) * 210;   // Q6_K
    const int idx = (int)(i & 255), h = idx >> 7, l = idx & 127;
    const uint32_t ql = (b[h * 64 + (l & 63)] >> ((l >> 6) * 4)) & 15u;
    const uint32_t qh = (b[128 + h * 32 + (l & 31)] >> ((l >> 5) * 2)) & 3u;
    const int sc = (int8_t)b[192 + (idx >> 4)];
    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(b[208] | (b[209] << 8)));
    const float ds = d * (float)sc;
    return ds * (float)((int)(ql | (qh << 4)) - 32);
}

// op 0 (resident_math.comp:30-32): column c of table row id.  An id past the
// vocabulary gives 0 and raises RTA_DEVERR_TOKEN (from column 0).
__device__ __forceinline__ float embed_value(int fmt, const uint8_t* __restrict__ table, int64_t row_bytes,
                                             int vocab, uint32_t id, int c) {
    if (id < (uint32_t)vocab) return dequant_value(fmt, table + (int64_t)id * row_bytes, c);
    if (c == 0) raise_error(RTA_DEVERR_TOKEN);
    return 0.0f;
}

// Stable logistic of resident_common.glsl:138 (detectorSigmoid).
__device__ __forceinline__ float detector_sigmoid(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float light = expf(v);
    return light / (1.0f + light);
}

__device__ __forceinline__ float signf(float v) { return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f); }

// sign(g) sign(u) |g| |u| sigmoid(g): the fused gate/up detector of
// resident_math.comp:71 (equal to SiLU(g) * u).
__device__ __forceinline__ float swiglu(float g, float u) {
    const float amplitude = fabsf(g) * fabsf(u) * detector_sigmoid(g);
    return signf(g) * signf(u) * amplitude;
}

// Host: calls f(std::integral_constant<int, NS>{}) with the smallest NS in {1, 2, 4, 8,
// 16} that covers nslab, or NS = 0 (plain loop) above 16.
template <class F>
inline void with_slab_count(int nslab, F&& f) {
    if (nslab <= 1) f(std::integral_constant<int, 1>{});
    else if (nslab <= 2) f(std::integral_constant<int, 2>{});
    else if (nslab <= 4) f(std::integral_constant<int, 4>{});
    else if (nslab <= 8) f(std::integral_constant<int, 8>{});
    else if (nslab <= 16) f(std::integral_constant<int, 16>{});
    else f(std::integral_constant<int, 0>{});
}

}  // namespace rta
