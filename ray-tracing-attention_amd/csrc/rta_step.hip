// rta_step.hip -- the rest of a decoder step around the projections and attention:
// embedding gather, RMSNorm, per-head norms, the gated delta-net recurrent layer
// (gates, short convolution, state update) and the history packer (gfx950).
#include <math.h>

#include "rta_common.hpp"
#include "rta_host.hpp"
#include "rta_internal.hpp"
#include "rta_pack.hpp"

namespace rta {

__device__ __forceinline__ float wave_sum(float v) { return wave_sum_dpp(v); }
// Sum over the 32 lanes of each half of a wave, every lane getting its half's sum: DPP
// steps inside each 16-lane row, then the row swap (lane ^ 16).
__device__ __forceinline__ float half_sum_dpp(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
    return add_xor16(v);
}
// The recurrent state's words held by one lane (float2 or float4 of one value row).
__device__ __forceinline__ float dot(float2 a, float2 b) { return a.x * b.x + a.y * b.y; }
__device__ __forceinline__ float dot(float4 a, float4 b) { return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w); }
__device__ __forceinline__ void scale_by(float2& s, float c) {
    s.x *= c;
    s.y *= c;
}
__device__ __forceinline__ void scale_by(float4& s, float c) {
    s.x *= c;
    s.y *= c;
    s.z *= c;
    s.w *= c;
}
__device__ __forceinline__ void axpy(float2& s, float f, float2 k) {   // s += f k
    s.x += f * k.x;
    s.y += f * k.y;
}
__device__ __forceinline__ void axpy(float4& s, float f, float4 k) {
    s.x += f * k.x;
    s.y += f * k.y;
    s.z += f * k.z;
    s.w += f * k.w;
}
__device__ __forceinline__ void store_nt(float2* p, float2 v) {
    using f2v = float __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(f2v{v.x, v.y}, reinterpret_cast<f2v*>(p));
}
__device__ __forceinline__ void store_nt(float4* p, float4 v) {
    using f4v = float __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(f4v{v.x, v.y, v.z, v.w}, reinterpret_cast<f4v*>(p));
}

// Sum over a block of NW waves through LDS red[NW]; every thread gets the total.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float silu(float v) { return v * detector_sigmoid(v); }

// ------------------------------------------------------------- embedding ----
// op 0 (resident_math.comp:30-32): out[b, c] = decoded table row ids[b].  Ids past
// the vocabulary give zeros and raise RTA_DEVERR_TOKEN.
__global__ void __launch_bounds__(256) embed_kernel(int fmt, const uint8_t* __restrict__ table, int64_t row_bytes,
                                                    int vocab, int hidden, const uint32_t* __restrict__ ids,
                                                    float* __restrict__ out) {
    const int b = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    if (c >= hidden) return;
    out[(int64_t)b * hidden + c] = embed_value(fmt, table, row_bytes, vocab, ids[b], c);
}

// --------------------------------------------------------------- RMSNorm ----
// op 1 (resident_math.comp:33-38): out = x * w / sqrt(mean(x^2) + eps), one block per row.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      int width, float eps, float* __restrict__ out) {
    __shared__ float red[4];
    const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)blockIdx.x * width);
    const int n4 = width >> 2;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n4; i += 256) {
        const float4 v = xr[i];
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum<4>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)width + eps);
    float4* o = reinterpret_cast<float4*>(out + (int64_t)blockIdx.x * width);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    for (int i = threadIdx.x; i < n4; i += 256) {
        const float4 v = xr[i], g = w4[i];
        o[i] = float4{v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w};
    }
}

// Split-K residual add fused with the next RMSNorm (decode step): one 1024-thread
// block per row; every thread keeps its float4 of the row in registers.
__global__ void __launch_bounds__(1024) residual_rmsnorm_kernel(float* __restrict__ hidden,
                                                                const float* __restrict__ part, int nslab,
                                                                const float* __restrict__ w, int width, float eps,
                                                                float* __restrict__ out) {
    __shared__ float red[16];
    constexpr int kMaxPer = 4;   // float4s per thread: width <= 16384
    const int b = blockIdx.x, n4 = width >> 2;
    float4* hr = reinterpret_cast<float4*>(hidden + (int64_t)b * width);
    float4 h[kMaxPer];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
        const int i = threadIdx.x + 1024 * j;
        if (i < n4) {
            float4 v = hr[i];
#pragma unroll 4
            for (int k = 0; k < nslab; ++k) {
                const float4 p = reinterpret_cast<const float4*>(part + ((int64_t)k * 32 + b) * width)[i];
                v.x += p.x;
                v.y += p.y;
                v.z += p.z;
                v.w += p.w;
            }
            if (nslab > 0) hr[i] = v;
            h[j] = v;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    }
    ss = block_sum<16>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)width + eps);
    float4* o = reinterpret_cast<float4*>(out + (int64_t)b * width);
    const float4* w4 = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
        const int i = threadIdx.x + 1024 * j;
        if (i < n4) {
            const float4 v = h[j], g = w4[i];
            o[i] = float4{v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w};
        }
    }
}

int residual_rmsnorm(float* hidden, const float* part, int nslab, const float* w, int batch, int width, float eps,
                     float* out, hipStream_t s) {
    if (!hidden || !w || !out || (nslab > 0 && !part)) return RTA_ERR_NULL;
    if (batch <= 0 || batch > 32 || width <= 0 || width % 4 || width > 4 * 1024 * 4 || nslab < 0) return RTA_ERR_SHAPE;
    if (!host::aligned(hidden, 16) || !host::aligned(w, 16) || !host::aligned(out, 16) ||
        (part && !host::aligned(part, 16)))
        return RTA_ERR_ALIGN;
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(batch), dim3(1024), 0, s, hidden, part, nslab, w, width, eps, out);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

// The residual add of residual_rmsnorm_kernel with the normalisation deferred to the
// readouts: block (column chunk c of 1024, row b) adds the K slabs, writes hidden and
// out = hidden * w, and the chunk's sum of squares to ss[4 b + c] (the four entries of
// a row, unused ones zero).  The row total is never needed here, so a row of up to
// 4096 columns spreads over up to 4 blocks.
constexpr int kNormChunk = 1024;

// NS: the slab loads in flight, NS >= nslab (1, 2, 4, 8, 16; every slab's load issued at
// once, indexes past the last slab clamped to it and not added), or 0 for a loop over more
// than 16 slabs.  The partials are added in slab order either way.
template <int NS>
__global__ void __launch_bounds__(256) residual_norm_deferred_kernel(float* __restrict__ hidden,
                                                                     const float* __restrict__ part, int nslab,
                                                                     const float* __restrict__ w, int width,
                                                                     float* __restrict__ out, float* __restrict__ ss) {
    __shared__ float red[4];
    const int c = blockIdx.x, b = blockIdx.y, n4 = width >> 2;
    const int i = c * (kNormChunk / 4) + threadIdx.x;
    float sq = 0.0f;
    if (i < n4) {
        float4* hr = reinterpret_cast<float4*>(hidden + (int64_t)b * width);
        float4 v = hr[i];
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
        reinterpret_cast<float4*>(out + (int64_t)b * width)[i] = float4{v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w};
    }
    sq = block_sum<4>(sq, red);
    if (threadIdx.x == 0) {
        ss[4 * b + c] = sq;
        if (c == 0)
            for (int z = gridDim.x; z < 4; ++z) ss[4 * b + z] = 0.0f;
    }
}

int residual_norm_deferred(float* hidden, const float* part, int nslab, const float* w, int batch, int width,
                           float* out, float* ss, hipStream_t s) {
    if (!hidden || !w || !out || !ss || (nslab > 0 && !part)) return RTA_ERR_NULL;
    if (batch <= 0 || batch > 32 || width <= 0 || width % 4 || width > 4 * kNormChunk || nslab < 0)
        return RTA_ERR_SHAPE;
    if (!host::aligned(ss, 16)) return RTA_ERR_ALIGN;
    if (!host::aligned(hidden, 16) || !host::aligned(w, 16) || !host::aligned(out, 16) ||
        (part && !host::aligned(part, 16)))
        return RTA_ERR_ALIGN;
    with_slab_count(nslab, [&](auto ns) {
        hipLaunchKernelGGL((residual_norm_deferred_kernel<decltype(ns)::value>),
                           dim3((width + kNormChunk - 1) / kNormChunk, batch), dim3(kNormChunk / 4), 0, s, hidden,
                           part, nslab, w, width, out, ss);
    });
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

// ------------------------------------------------------------- head norms ----
// ops 14 / 15 / 20 (resident_math.comp:113-115,139-140), in place: one wave per
// (row, head) of hd = 64 * VPL values:
//   x = x * w[h*hd+c] / sqrt(sum(x^2) / (mean ? hd : 1) + eps) * (gate ? g*sigmoid(g) : 1)
template <int VPL>
__global__ void __launch_bounds__(256) head_norm_kernel(float* __restrict__ x, int x_stride,
                                                        const float* __restrict__ w, const float* __restrict__ gate,
                                                        int gate_stride, int heads, int mean, float eps) {
    const int lane = threadIdx.x & 63;
    const int h = blockIdx.x * 4 + (threadIdx.x >> 6), r = blockIdx.y;
    if (h >= heads) return;
    constexpr int hd = 64 * VPL;
    float* xh = x + (int64_t)r * x_stride + (int64_t)h * hd;
    float v[VPL];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = xh[lane + 64 * i];
        ss += v[i] * v[i];
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf((mean ? ss / (float)hd : ss) + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int c = lane + 64 * i;
        float o = v[i] * inv;
        if (w) o *= w[h * hd + c];
        if (gate) o *= silu(gate[(int64_t)r * gate_stride + (int64_t)h * hd + c]);
        xh[c] = o;
    }
}

// -------------------------------------------------------- delta-net gates ----
// op 18 (resident_math.comp:131-133) after its two projections:
// decay = exp(-exp(a_log[h]) * softplus(a + dt_bias[h])), beta = sigmoid(b).
__global__ void __launch_bounds__(256) delta_gates_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                          int stride, const float* __restrict__ a_log,
                                                          const float* __restrict__ dt_bias, int batch, int heads,
                                                          float* __restrict__ decay, float* __restrict__ beta) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= batch * heads) return;
    const int r = i / heads, h = i - r * heads;
    const float av = a[(int64_t)r * stride + h] + dt_bias[h];
    const float sp = fmaxf(av, 0.0f) + log1pf(expf(-fabsf(av)));   // softplus, resident_common.glsl:80
    decay[i] = expf(-expf(a_log[h]) * sp);
    beta[i] = detector_sigmoid(b[(int64_t)r * stride + h]);
}

// ---------------------------------------------------- short convolution ----
// ops 19 + 20 (resident_math.comp:134-140) for one new token per sequence: block
// (head, sequence), thread c of hd.  For each part (q, k, v) coordinate
// p = part*W + h*hd + c:  s = sum_j<3 w[p][j] state[p][j] + w[p][3] raw[p];
// y = s * sigmoid(s); the window shifts by one; q and k are L2-normalised per head.
__global__ void __launch_bounds__(128) short_conv_kernel(const float* __restrict__ raw, int raw_stride,
                                                         float* __restrict__ state, const float* __restrict__ w,
                                                         int heads, float eps, float* __restrict__ out) {
    __shared__ float red[2];
    const int h = blockIdx.x, b = blockIdx.y, c = threadIdx.x, hd = 128;
    const int W = heads * hd, W3 = 3 * W;
    float y[3];
#pragma unroll
    for (int part = 0; part < 3; ++part) {
        const int p = part * W + h * hd + c;
        float* st = state + ((int64_t)b * W3 + p) * 3;
        const float4 wp = *reinterpret_cast<const float4*>(w + (int64_t)p * 4);
        const float x = raw[(int64_t)b * raw_stride + p];
        const float s0 = st[0], s1 = st[1], s2 = st[2];
        const float s = wp.x * s0 + wp.y * s1 + wp.z * s2 + wp.w * x;
        y[part] = silu(s);
        st[0] = s1;
        st[1] = s2;
        st[2] = x;
    }
#pragma unroll
    for (int part = 0; part < 2; ++part) {
        float ss = wave_sum(y[part] * y[part]);
        __syncthreads();
        if ((c & 63) == 0) red[c >> 6] = ss;
        __syncthreads();
        y[part] *= 1.0f / sqrtf(red[0] + red[1] + eps);
    }
#pragma unroll
    for (int part = 0; part < 3; ++part) out[(int64_t)b * W3 + part * W + h * hd + c] = y[part];
}

// ---------------------------------------------------------- delta rule ----
// op 21 / resident_state.comp, one token per sequence: block (head, sequence), 4
// waves x 32 value rows of the hd x hd state ([value][key]); lane l holds keys 2l,
// 2l+1.  Per row:  s = decay s;  u = s.k;  s += beta (v - u) k;  o = s.q / sqrt(hd).
// A wave issues the loads of all its 32 rows at once (one memory round trip per
// block), and the 64 row sums go through DPP steps inside each 16-lane row plus two
// cross-row shuffles.  With norm_w the gated RMSNorm of op 15 (resident_math.comp:115)
// is applied to o.
__global__ void __launch_bounds__(256) delta_rule_kernel(float* __restrict__ state, const float* __restrict__ qkv,
                                                         int qkv_stride, const float* __restrict__ decay,
                                                         const float* __restrict__ beta, int heads,
                                                         const float* __restrict__ norm_w,
                                                         const float* __restrict__ gate, int gate_stride, float eps,
                                                         float* __restrict__ out, int out_stride) {
    constexpr int hd = 128, kRows = hd / 4;
    __shared__ float o_s[hd];
    __shared__ float red[4];
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = heads * hd;
    const float* row = qkv + (int64_t)b * qkv_stride;
    float2* S = reinterpret_cast<float2*>(state + ((int64_t)b * heads + h) * hd * hd) + wave * kRows * (hd / 2) + lane;
    float2 s[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) s[i] = S[i * (hd / 2)];
    const float2 q = *reinterpret_cast<const float2*>(row + h * hd + 2 * lane);
    const float2 k = *reinterpret_cast<const float2*>(row + W + h * hd + 2 * lane);
    const float* vv = row + 2 * W + h * hd + wave * kRows;   // this wave's value coordinates (uniform)
    const float dc = decay[(int64_t)b * heads + h], bt = beta[(int64_t)b * heads + h];
    const float scale = 1.0f / sqrtf((float)hd);
    float u[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        s[i].x *= dc;
        s[i].y *= dc;
        u[i] = wave_sum_dpp(s[i].x * k.x + s[i].y * k.y);
    }
    float o[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        const float delta = bt * (vv[i] - u[i]);
        s[i].x += delta * k.x;
        s[i].y += delta * k.y;
        S[i * (hd / 2)] = s[i];
        o[i] = s[i].x * q.x + s[i].y * q.y;
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) o[i] = wave_sum_dpp(o[i]);
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < kRows; ++i) o_s[wave * kRows + i] = o[i] * scale;
    }
    __syncthreads();
    float* op = out + (int64_t)b * out_stride + h * hd;
    if (!norm_w) {
        if (threadIdx.x < hd) op[threadIdx.x] = o_s[threadIdx.x];
        return;
    }
    const float v = threadIdx.x < hd ? o_s[threadIdx.x] : 0.0f;
    const float ss = block_sum<4>(v * v, red);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    if (threadIdx.x < hd) {
        const float g = gate[(int64_t)b * gate_stride + h * hd + threadIdx.x];
        op[threadIdx.x] = v * inv * norm_w[h * hd + threadIdx.x] * silu(g);
    }
}

// ------------------------------------------- recurrent layer, fused middle ----
// The middle of a recurrent layer for one (head, sequence) in one block, with the
// arithmetic of delta_gates_kernel, short_conv_kernel and delta_rule_kernel:
//   the head's in-projection rows (q | k | v | z | a | b of the layer) summed over
//   the packed readout's K slabs in slab order (as gemm_reduce_kernel adds them);
//   gates (op 18); short convolution + SiLU + L2 norm of q and k (ops 19, 20); the
//   delta rule (op 21) and the gated RMSNorm (op 15).
// Row r of sequence b is sum_k proj[k * slab_stride + b * row_stride + r], k < nslab.
// q and k hold key_heads heads (KW = key_heads hd rows each): head h reads head
// h % key_heads, while the convolution runs over the heads' own channels (weights and
// window of channel part W + h hd + c).  With ext_a, the gate inputs are ext_a[b
// ext_stride + h] and ext_b[...] times the row's RMSNorm factor rn (1 without rn).
template <int NS, int NW>
__global__ void __launch_bounds__(64 * NW) recurrent_mix_kernel(
    const float* __restrict__ proj, int64_t slab_stride, int row_stride, int nslab, int key_heads,
    const float* __restrict__ ext_a, const float* __restrict__ ext_b, int ext_stride, const RowNorm rn,
    float* __restrict__ conv_state, const float* __restrict__ conv_w, const float* __restrict__ a_log,
    const float* __restrict__ dt_bias, float* __restrict__ state, const float* __restrict__ norm_w, int heads,
    float eps, float* __restrict__ out, int out_stride) {
    constexpr int hd = 128, kRows = hd / NW;   // state rows per wave
    __shared__ __align__(16) float qkv_s[3][hd];
    __shared__ float z_s[hd];
    __shared__ float gates_s[2];
    __shared__ float o_s[hd];
    __shared__ float red[NW];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int W = heads * hd, W3 = 3 * W, KW = key_heads * hd, hk = h % key_heads;
    const int row_v = 2 * KW, row_z = row_v + W, row_a = row_z + W;
    const float* src = proj + (int64_t)b * row_stride;
    // in-projection rows: every slab load is issued at once (indices clamped to the
    // last slab, which is not added twice), then summed in slab order
    auto load_row = [&](int r, float t[NS]) {
#pragma unroll
        for (int k = 0; k < NS; ++k) t[k] = src[(int64_t)min(k, nslab - 1) * slab_stride + r];
    };
    auto sum_row = [&](const float t[NS]) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < NS; ++k)
            if (k < nslab) v += t[k];
        return v;
    };
    // threads 0..127: coordinate c of q, k, v (ops 19, 20); 128..255: the gate z, and
    // thread 128 the decay / beta inputs (op 18); threads from 256 on only hold state.  Their loads go out before the
    // recurrent state's, which take the longest and complete in order behind them.
    const int c = tid & (hd - 1);
    const bool conv = tid < hd;
    float raw[3][NS], ab[2][NS];
    float4 wp[3];
    float sv[3][3];
    if (conv) {
#pragma unroll
        for (int part = 0; part < 3; ++part) {
            const int pc = part * W + h * hd + c;   // the channel; its input row:
            load_row(part < 2 ? part * KW + hk * hd + c : row_v + h * hd + c, raw[part]);
            wp[part] = *reinterpret_cast<const float4*>(conv_w + (int64_t)pc * 4);
            const float* st = conv_state + ((int64_t)b * W3 + pc) * 3;
            sv[part][0] = st[0];
            sv[part][1] = st[1];
            sv[part][2] = st[2];
        }
    } else if (tid < 2 * hd) {
        load_row(row_z + h * hd + c, raw[0]);
        if (!ext_a) {
            load_row(row_a + h, ab[0]);
            load_row(row_a + heads + h, ab[1]);
        }
    }
    asm volatile("" ::: "memory");   // the state loads stay behind the loads above
    // The wave's value rows: lane l holds keys 2 l, 2 l + 1 of every row (float2 words),
    // or, with no K slabs to add (NS = 1: registers to spare within the 64 VGPRs of two
    // blocks per CU), keys 4 (l % 32) .. + 3 of the rows 2 j + l / 32 (float4 words: one
    // load covers two rows, and the row sums take half-wave reductions; batch-1 step
    // 1.929 -> 1.899 ms, while at 4 K slabs the wider words cost 67 VGPRs and half the
    // blocks per CU).  Word j of the lane is value row rbase + j rstep.
    constexpr bool kWide = NS == 1;
    using Word = typename std::conditional<kWide, float4, float2>::type;
    constexpr int kWords = kWide ? kRows / 2 : kRows, rstep = kWide ? 2 : 1, kw = kWide ? 4 : 2;
    const int half = kWide ? lane >> 5 : 0, cl = kWide ? lane & 31 : lane;
    const int rbase = wave * kRows + half;
    Word* S = reinterpret_cast<Word*>(state + ((int64_t)b * heads + h) * hd * hd + (int64_t)rbase * hd) + cl;
    Word s[kWords];
#pragma unroll
    for (int j = 0; j < kWords; ++j) s[j] = S[j * (hd / 2)];   // (hd / 2 words: rstep rows)

    float y[3] = {0.0f, 0.0f, 0.0f};
    if (conv) {
#pragma unroll
        for (int part = 0; part < 3; ++part) {
            const int pc = part * W + h * hd + c;
            const float x = sum_row(raw[part]);
            const float v = wp[part].x * sv[part][0] + wp[part].y * sv[part][1] + wp[part].z * sv[part][2] +
                            wp[part].w * x;
            y[part] = silu(v);
            float* st = conv_state + ((int64_t)b * W3 + pc) * 3;
            st[0] = sv[part][1];
            st[1] = sv[part][2];
            st[2] = x;
        }
    } else if (tid < 2 * hd) {
        z_s[c] = sum_row(raw[0]);
        if (c == 0) {
            float ga, gb;
            if (ext_a) {
                const float f = rn.part ? row_norm_factor(rn, rn.part[b]) : 1.0f;
                ga = ext_a[(int64_t)b * ext_stride + h] * f;
                gb = ext_b[(int64_t)b * ext_stride + h] * f;
            } else {
                ga = sum_row(ab[0]);
                gb = sum_row(ab[1]);
            }
            const float av = ga + dt_bias[h];
            const float sp = fmaxf(av, 0.0f) + log1pf(expf(-fabsf(av)));   // softplus, resident_common.glsl:80
            gates_s[0] = expf(-expf(a_log[h]) * sp);
            gates_s[1] = detector_sigmoid(gb);
        }
    }
    // L2 norm of q and k over the head (waves 0 and 1 hold its 128 coordinates)
#pragma unroll
    for (int part = 0; part < 2; ++part) {
        const float ss = wave_sum(y[part] * y[part]);
        __syncthreads();
        if (lane == 0 && wave < 2) red[wave] = ss;
        __syncthreads();
        y[part] *= 1.0f / sqrtf(red[0] + red[1] + eps);
    }
    if (tid < hd) {
#pragma unroll
        for (int part = 0; part < 3; ++part) qkv_s[part][tid] = y[part];
    }
    __syncthreads();

    // op 21 over the lane's words (the updated state is stored non-temporally: it is
    // read again only by the next step, after every other layer's weights have passed
    // through the caches)
    const Word q = *reinterpret_cast<const Word*>(&qkv_s[0][kw * cl]);
    const Word k = *reinterpret_cast<const Word*>(&qkv_s[1][kw * cl]);
    const float* vv = &qkv_s[2][rbase];
    const float dc = gates_s[0], bt = gates_s[1];
    const float scale = 1.0f / sqrtf((float)hd);
    auto row_sum = [](float v) { return kWide ? half_sum_dpp(v) : wave_sum_dpp(v); };
    float u[kWords];
#pragma unroll
    for (int j = 0; j < kWords; ++j) {
        scale_by(s[j], dc);
        u[j] = row_sum(dot(s[j], k));
    }
    float o[kWords];
#pragma unroll
    for (int j = 0; j < kWords; ++j) {
        axpy(s[j], bt * (vv[j * rstep] - u[j]), k);
        store_nt(S + j * (hd / 2), s[j]);
        o[j] = dot(s[j], q);
    }
#pragma unroll
    for (int j = 0; j < kWords; ++j) o[j] = row_sum(o[j]);
    if (cl == 0) {
#pragma unroll
        for (int j = 0; j < kWords; ++j) o_s[rbase + j * rstep] = o[j] * scale;
    }
    __syncthreads();
    // op 15: gated RMSNorm of o
    const float v = tid < hd ? o_s[tid] : 0.0f;
    const float ss = block_sum<NW>(v * v, red);
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    if (tid < hd) out[(int64_t)b * out_stride + h * hd + tid] = v * inv * norm_w[h * hd + tid] * silu(z_s[tid]);
}

int recurrent_mix(const float* proj, int64_t slab_stride, int row_stride, int nslab, int key_heads, const float* ext_a,
                  const float* ext_b, int ext_stride, const RowNorm& rn, float* conv_state, const float* conv_w,
                  const float* a_log, const float* dt_bias, float* state, const float* norm_w, int batch, int heads,
                  float eps, float* out, int out_stride, hipStream_t s) {
    if (!proj || !conv_state || !conv_w || !a_log || !dt_bias || !state || !norm_w || !out) return RTA_ERR_NULL;
    if ((ext_a == nullptr) != (ext_b == nullptr)) return RTA_ERR_NULL;
    if (key_heads <= 0 || key_heads > heads) return RTA_ERR_RANGE;
    const int rows = 2 * key_heads * 128 + 2 * heads * 128 + (ext_a ? 0 : 2 * heads);
    if (batch <= 0 || heads <= 0 || nslab <= 0 || row_stride < rows || (ext_a && ext_stride < heads))
        return RTA_ERR_SHAPE;
    if (nslab > 16) return RTA_ERR_RANGE;
    // 16 waves per (sequence, head) block, 8 state rows each: the per-row reductions of
    // a head run in parallel, and at large batches the state reads of one block overlap
    // the state writes of another (measured faster than 4 waves x 32 rows at batch 1 and 32)
    constexpr int kWaves = 16;
    const dim3 g(heads, batch), blk(64 * kWaves);
#define RTA_MIX(NS) hipLaunchKernelGGL((recurrent_mix_kernel<NS, kWaves>), g, blk, 0, s, proj, slab_stride, \
                                       row_stride, nslab, key_heads, ext_a, ext_b, ext_stride, rn, conv_state, conv_w, \
                                       a_log, dt_bias, state, norm_w, heads, eps, out, out_stride)
    if (nslab == 1) RTA_MIX(1);
    else if (nslab == 2) RTA_MIX(2);
    else if (nslab <= 4) RTA_MIX(4);
    else if (nslab <= 8) RTA_MIX(8);
    else RTA_MIX(16);
#undef RTA_MIX
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

// --------------------------------------------------------- history packer ----
// op 34 (resident_history_quant.glsl:9-41): block (j, b) quantises superblock j (values
// 256 j .. 256 j + 255) of sequence b's new key and value rows with the shared packer
// routine (rta_pack.hpp, the arithmetic the decode step's middle kernel runs as well)
// and writes it to packet slot slot[b]; block j = 0 also zeroes the packet's padding.
constexpr int kPackMaxBlocks = 16;   // kvw <= 4096

__global__ void __launch_bounds__(256) pack_history_kernel(const float* __restrict__ kin, int k_stride,
                                                           const float* __restrict__ vin, int v_stride, int kvw,
                                                           int fmt_k, int fmt_v, const int64_t* __restrict__ slot,
                                                           int64_t n_slots, int64_t stride,
                                                           uint8_t* __restrict__ packets) {
    __shared__ float xs[2][256];   // the superblock of the K and V rows, zero past kvw
    __shared__ PackScratch st[2];
    __shared__ uint8_t fb[2][212];
    const int j = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int nsb = gridDim.x, c = 256 * j + tid;
    const float k = c < kvw ? kin[(int64_t)b * k_stride + c] : 0.0f;
    const float v = c < kvw ? vin[(int64_t)b * v_stride + c] : 0.0f;
    xs[0][tid] = k;
    xs[1][tid] = v;
    __syncthreads();
    const bool q4[2] = {fmt_k == RTA_Q4_K, fmt_v == RTA_Q4_K};
    pack_superblock_pair(xs, q4, st, fb, tid);
    const int64_t s = slot[b];
    if (s < 0 || s >= n_slots) {
        if (tid == 0 && j == 0) raise_error(RTA_DEVERR_HITS);
        return;
    }
    uint8_t* pk = packets + s * stride;
    const int kb = q4[0] ? 144 : 210, vb = q4[1] ? 144 : 210;
    const int64_t v_offset = (int64_t)nsb * kb;
    if (tid < kb) pk[(int64_t)j * kb + tid] = fb[0][tid];
    if (tid < vb) pk[v_offset + (int64_t)j * vb + tid] = fb[1][tid];
    if (j == 0)   // the packet's padding to 8 bytes
        for (int64_t i = v_offset + (int64_t)nsb * vb + tid; i < stride; i += 256) pk[i] = 0;
}

}  // namespace rta

using namespace rta;

extern "C" {

int rta_embed(int fmt, const void* table, int vocab, int hidden, const uint32_t* ids, int batch, float* out,
              rta_stream_t stream) {
    int64_t rb = 0;
    const int rc = host::embed_args(fmt, table, vocab, hidden, ids, batch, out, &rb);
    if (rc) return rc;
    hipLaunchKernelGGL(embed_kernel, dim3((hidden + 255) / 256, batch), dim3(256), 0, (hipStream_t)stream, fmt,
                       static_cast<const uint8_t*>(table), rb, vocab, hidden, ids, out);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_rmsnorm(const float* x, const float* w, int rows, int width, float eps, float* out, rta_stream_t stream) {
    if (!x || !w || !out) return RTA_ERR_NULL;
    if (rows <= 0 || width <= 0 || width % 4) return RTA_ERR_SHAPE;
    if (!(eps >= 0.0f)) return RTA_ERR_RANGE;
    if (!host::aligned(x, 16) || !host::aligned(w, 16) || !host::aligned(out, 16)) return RTA_ERR_ALIGN;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, (hipStream_t)stream, x, w, width, eps, out);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_head_norm(float* x, int x_stride, const float* w, const float* gate, int gate_stride, int rows, int heads,
                  int hd, int mean, float eps, rta_stream_t stream) {
    if (!x) return RTA_ERR_NULL;
    if (rows <= 0 || heads <= 0 || x_stride < heads * hd || (gate && gate_stride < heads * hd)) return RTA_ERR_SHAPE;
    if ((hd != 64 && hd != 128 && hd != 256) || !(eps >= 0.0f)) return RTA_ERR_RANGE;
    const dim3 g((heads + 3) / 4, rows), bl(256);
    hipStream_t s = (hipStream_t)stream;
    if (hd == 64) hipLaunchKernelGGL(head_norm_kernel<1>, g, bl, 0, s, x, x_stride, w, gate, gate_stride, heads, mean, eps);
    else if (hd == 128) hipLaunchKernelGGL(head_norm_kernel<2>, g, bl, 0, s, x, x_stride, w, gate, gate_stride, heads, mean, eps);
    else hipLaunchKernelGGL(head_norm_kernel<4>, g, bl, 0, s, x, x_stride, w, gate, gate_stride, heads, mean, eps);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_delta_gates(const float* a, const float* b, int stride, const float* a_log, const float* dt_bias, int batch,
                    int heads, float* decay, float* beta, rta_stream_t stream) {
    if (!a || !b || !a_log || !dt_bias || !decay || !beta) return RTA_ERR_NULL;
    if (batch <= 0 || heads <= 0 || stride < heads) return RTA_ERR_SHAPE;
    const int n = batch * heads;
    hipLaunchKernelGGL(delta_gates_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, a, b, stride,
                       a_log, dt_bias, batch, heads, decay, beta);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_short_conv(const float* raw, int raw_stride, float* state, const float* w, int batch, int heads, int hd,
                   float eps, float* out, rta_stream_t stream) {
    if (!raw || !state || !w || !out) return RTA_ERR_NULL;
    if (batch <= 0 || heads <= 0 || raw_stride < 3 * heads * hd) return RTA_ERR_SHAPE;
    if (hd != 128 || !(eps >= 0.0f)) return RTA_ERR_RANGE;
    if (!host::aligned(w, 16)) return RTA_ERR_ALIGN;
    hipLaunchKernelGGL(short_conv_kernel, dim3(heads, batch), dim3(128), 0, (hipStream_t)stream, raw, raw_stride,
                       state, w, heads, eps, out);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_delta_rule(float* state, const float* qkv, int qkv_stride, const float* decay, const float* beta, int batch,
                   int heads, int hd, const float* norm_w, const float* gate, int gate_stride, float eps, float* out,
                   int out_stride, rta_stream_t stream) {
    if (!state || !qkv || !decay || !beta || !out || (norm_w && !gate)) return RTA_ERR_NULL;
    if (batch <= 0 || heads <= 0 || qkv_stride < 3 * heads * hd || out_stride < heads * hd ||
        (gate && gate_stride < heads * hd))
        return RTA_ERR_SHAPE;
    if (hd != 128 || !(eps >= 0.0f)) return RTA_ERR_RANGE;
    if (!host::aligned(state, 16) || !host::aligned(qkv, 8) || qkv_stride % 2) return RTA_ERR_ALIGN;
    hipLaunchKernelGGL(delta_rule_kernel, dim3(heads, batch), dim3(256), 0, (hipStream_t)stream, state, qkv,
                       qkv_stride, decay, beta, heads, norm_w, gate, gate_stride, eps, out, out_stride);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_pack_history(const float* k, int k_stride, const float* v, int v_stride, int batch, int kvw, int fmt_k,
                     int fmt_v, const int64_t* slot, int64_t n_slots, void* packets, rta_stream_t stream) {
    if (!k || !v || !slot || !packets) return RTA_ERR_NULL;
    // a packet holds one Q4_K and one Q6_K field (354 bytes per 256 coordinates)
    if ((fmt_k != RTA_Q4_K && fmt_k != RTA_Q6_K) || (fmt_v != RTA_Q4_K && fmt_v != RTA_Q6_K) || fmt_k == fmt_v)
        return RTA_ERR_FORMAT;
    if (batch <= 0 || kvw <= 0 || k_stride < kvw || v_stride < kvw || n_slots <= 0) return RTA_ERR_SHAPE;
    if (kvw > 256 * kPackMaxBlocks) return RTA_ERR_RANGE;
    const int64_t stride = host::history_bytes(kvw);
    if (!host::aligned(packets, 8)) return RTA_ERR_ALIGN;
    hipLaunchKernelGGL(pack_history_kernel, dim3((kvw + 255) / 256, batch), dim3(256), 0, (hipStream_t)stream, k,
                       k_stride, v, v_stride, kvw, fmt_k, fmt_v, slot, n_slots, stride,
                       static_cast<uint8_t*>(packets));
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

}  // extern "C"
