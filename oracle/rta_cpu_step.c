/*
 * rta_cpu_step.c -- one greedy decode step of the hybrid decoder on the host CPU, in
 * fp32 with OpenMP: the timed CPU baseline of the decode-step benchmark, and a second,
 * independent composition of the step the tests compare with the fp64 one.
 *
 * TEST INFRASTRUCTURE ONLY (the checker / the CPU baseline).  Only tests/ and
 * bench.py's cpu_baseline leg load this library; the product library never does.
 *
 * The step follows the reference worker's layer sequence (Resident::forward / layer /
 * word, ray_tracing/native/src/optical_resident.cpp:455-530) for a batch of
 * independent sequences, with the ops of resident_math.comp: embedding (op 0,
 * :30-32), RMSNorm (op 1, :33-38), projections (op 2, :39-75), SwiGLU (:54-58,71),
 * QK-norm (op 14, :113-114), RoPE (op 3, :76-77; phase resident_common.glsl:117),
 * history packing (op 34, resident_history_quant.glsl:9-41), attention
 * (resident_ray.comp:56-76), delta-net gates, short convolution, delta rule and the
 * gated norm (ops 18-21 and 15, :131-148; resident_state.comp), the LM head and the
 * argmax (:117-130).  Weights are GGUF rows; values are dequantised with the
 * reference's fp32 op order, products are summed in fp32 (8-wide vector lanes).
 */
#include "rta_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#endif

/* ---- row decoding (resident_quant.glsl:6-20), as orc_dequant ---------------------- */
static void decode_row(int fmt, const uint8_t* row, int cols, float* out) { orc_dequant(fmt, row, cols, out); }

static float dot(const float* a, const float* b, int n) {
#if defined(__AVX2__) && defined(__FMA__)
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps(), s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), s1);
        s2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), s2);
        s3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), s3);
    }
    __m256 s = _mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3));
    float t[8];
    _mm256_storeu_ps(t, s);
    float r = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    for (; i < n; ++i) r += a[i] * b[i];
    return r;
#else
    float s[8] = {0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; ++j) s[j] += a[i + j] * b[i + j];
    float r = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
    for (; i < n; ++i) r += a[i] * b[i];
    return r;
#endif
}

/* y[b, r] (+)= sum_c W[r, c] x[b, c]: each row decoded once, then dotted with every
 * batch row (resident_math.comp:39-75; the matrixRows tile reuses a decode the same way). */
static void gemv(int fmt, const void* W, int rows, int cols, const float* x, int batch, float* y, int accumulate) {
    const int64_t rb = orc_row_bytes(fmt, cols);
    #pragma omp parallel
    {
        float* buf = (float*)malloc(sizeof(float) * (size_t)cols);
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            decode_row(fmt, (const uint8_t*)W + (int64_t)r * rb, cols, buf);
            for (int b = 0; b < batch; ++b) {
                const float v = dot(buf, x + (int64_t)b * cols, cols);
                float* dst = y + (int64_t)b * rows + r;
                *dst = accumulate ? *dst + v : v;
            }
        }
        free(buf);
    }
}

static float sigmoidf_stable(float v) {   /* resident_common.glsl:138 */
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

static void rmsnorm(const float* x, const float* w, int rows, int width, float eps, float* out) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (int64_t)r * width;
        const float inv = 1.0f / sqrtf(dot(xr, xr, width) / (float)width + eps);
        for (int c = 0; c < width; ++c) out[(int64_t)r * width + c] = xr[c] * inv * w[c];
    }
}

/* per head of hd values: x * w / sqrt(sum(x^2) / (mean ? hd : 1) + eps) */
static void head_norm(float* x, const float* w, int heads, int hd, int mean, float eps) {
    for (int h = 0; h < heads; ++h) {
        float* xh = x + (int64_t)h * hd;
        const float inv = 1.0f / sqrtf(dot(xh, xh, hd) / (mean ? (float)hd : 1.0f) + eps);
        for (int c = 0; c < hd; ++c) xh[c] = xh[c] * inv * (w ? w[h * hd + c] : 1.0f);
    }
}

static void rope(float* v, int heads, int hd, int rotary, int64_t t, double theta) {
    const int active = rotary / 2;
    for (int h = 0; h < heads; ++h)
        for (int p = 0; p < active; ++p) {
            const double phase = (double)t * pow(theta, -(double)p / (double)active);
            const double sn = sin(phase), cs = cos(phase);
            float* e = v + (int64_t)h * hd + 2 * p;
            const double a = e[0], b = e[1];
            e[0] = (float)(a * cs - b * sn);
            e[1] = (float)(a * sn + b * cs);
        }
}

/* One query over the history of a sequence: o = softmax(q k / sqrt(hd)) v. */
static void attend(const float* q, int hq, int hkv, int hd, const uint8_t* packets, int64_t stride, int64_t kv_off,
                   int fmt_k, int fmt_v, int64_t base, int64_t t, int64_t capacity, float* out, float* kbuf,
                   float* vbuf, float* scores) {
    const int kvw = hkv * hd, group = hq / hkv;
    const int64_t visible = t + 1 < capacity ? t + 1 : capacity;
    const int64_t nb = (kvw + 255) / 256;
    const float inv = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < hq; ++h) scores[(int64_t)h * visible] = -INFINITY;
    for (int64_t r = 0; r < visible; ++r) {
        const uint8_t* pk = packets + (base + (t - r) % capacity) * stride;
        decode_row(fmt_k, pk, (int)(nb * 256), kbuf);
        for (int h = 0; h < hq; ++h)
            scores[(int64_t)h * visible + r] = dot(q + (int64_t)h * hd, kbuf + (h / group) * hd, hd) * inv;
    }
    for (int h = 0; h < hq; ++h) {
        float* s = scores + (int64_t)h * visible;
        float mx = -INFINITY;
        for (int64_t r = 0; r < visible; ++r) mx = s[r] > mx ? s[r] : mx;
        float z = 0.0f;
        for (int64_t r = 0; r < visible; ++r) { s[r] = expf(s[r] - mx); z += s[r]; }
        for (int64_t r = 0; r < visible; ++r) s[r] /= (z > 1e-30f ? z : 1e-30f);
        for (int c = 0; c < hd; ++c) out[(int64_t)h * hd + c] = 0.0f;
    }
    for (int64_t r = 0; r < visible; ++r) {
        const uint8_t* pk = packets + (base + (t - r) % capacity) * stride;
        decode_row(fmt_v, pk + kv_off, (int)(nb * 256), vbuf);
        for (int h = 0; h < hq; ++h) {
            const float w = scores[(int64_t)h * visible + r];
            const float* vh = vbuf + (h / group) * hd;
            float* o = out + (int64_t)h * hd;
            for (int c = 0; c < hd; ++c) o[c] += w * vh[c];
        }
    }
}

static int is_full(const orc_step_model* m, int l) { return m->full_every > 0 && l % m->full_every == m->full_every - 1; }

int orc_step_f32(const orc_step_model* m, int batch, float* rec, float* conv, uint8_t* packets, int32_t* ctx,
                 uint32_t* tokens, float* logits_out, int threads) {
    if (!m || !rec || !conv || !packets || !ctx || !tokens || batch <= 0 || m->head_dim != 128) return 1;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
    const int D = m->hidden, hd = m->head_dim, hq = m->q_heads, hkv = m->kv_heads, H = m->rec_heads, S = H * hd;
    const int FF = m->ff, V = m->vocab, B = batch, kvw = hkv * hd;
    const int rows_full = (hq + 2 * hkv) * hd, rows_rec = 4 * S + 2 * H;
    const int64_t cap = m->capacity, pstride = orc_history_bytes(kvw);
    const int64_t nb = (kvw + 255) / 256, kv_off = nb * (m->fmt_k == ORC_Q4_K ? 144 : 210);
    const int maxrows = rows_full > rows_rec ? rows_full : rows_rec;
    float* x = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* n = (float*)malloc(sizeof(float) * (size_t)B * D);
    float* p = (float*)malloc(sizeof(float) * (size_t)B * maxrows);
    float* mix = (float*)malloc(sizeof(float) * (size_t)B * (hq * hd > S ? hq * hd : S));
    float* g = (float*)malloc(sizeof(float) * (size_t)B * FF);
    float* u = (float*)malloc(sizeof(float) * (size_t)B * FF);
    float* lg = logits_out ? logits_out : (float*)malloc(sizeof(float) * (size_t)B * V);
    if (!x || !n || !p || !mix || !g || !u || !lg) return 6;
    for (int b = 0; b < B; ++b)
        if (orc_embed(m->fmt_embed, m->embed, V, D, tokens + b, 1, x + (int64_t)b * D)) return 7;
    int lf = 0, lr = 0;
    for (int l = 0; l < m->layers; ++l) {
        const orc_step_layer* L = m->layers_ptr + l;
        rmsnorm(x, L->norm_in, B, D, m->eps, n);
        if (is_full(m, l)) {
            gemv(m->fmt_proj, L->w_in, rows_full, D, n, B, p, 0);
            uint8_t* pk = packets + (int64_t)lf * B * cap * pstride;
            #pragma omp parallel
            {
                float* kbuf = (float*)malloc(sizeof(float) * (size_t)(nb * 256));
                float* vbuf = (float*)malloc(sizeof(float) * (size_t)(nb * 256));
                float* sc = (float*)malloc(sizeof(float) * (size_t)hq * (size_t)cap);
                #pragma omp for schedule(dynamic)
                for (int b = 0; b < B; ++b) {
                    float* pr = p + (int64_t)b * rows_full;
                    const int64_t t = ctx[b];
                    head_norm(pr, L->q_norm, hq, hd, 1, m->eps);               /* op 14 */
                    head_norm(pr + hq * hd, L->k_norm, hkv, hd, 1, m->eps);
                    rope(pr, hq, hd, m->rope_rotary, t, m->rope_theta);         /* op 3 */
                    rope(pr + hq * hd, hkv, hd, m->rope_rotary, t, m->rope_theta);
                    orc_pack_history(pr + hq * hd, pr + (hq + hkv) * hd, kvw, m->fmt_k, m->fmt_v,   /* op 34 */
                                     pk + ((int64_t)b * cap + t % cap) * pstride);
                    attend(pr, hq, hkv, hd, pk, pstride, kv_off, m->fmt_k, m->fmt_v, (int64_t)b * cap, t, cap,
                           mix + (int64_t)b * hq * hd, kbuf, vbuf, sc);
                }
                free(kbuf); free(vbuf); free(sc);
            }
            gemv(m->fmt_proj, L->w_o, D, hq * hd, mix, B, x, 1);
            ++lf;
        } else {
            gemv(m->fmt_proj, L->w_in, rows_rec, D, n, B, p, 0);
            float* cs = conv + (int64_t)lr * B * 3 * S * 3;
            float* st = rec + (int64_t)lr * B * H * hd * hd;
            #pragma omp parallel for collapse(2) schedule(static)
            for (int b = 0; b < B; ++b)
                for (int h = 0; h < H; ++h) {
                    const float* pr = p + (int64_t)b * rows_rec;
                    /* op 18: gates */
                    const float av = pr[4 * S + h] + L->dt_bias[h], bv = pr[4 * S + H + h];
                    const float sp = (av > 0.0f ? av : 0.0f) + log1pf(expf(-fabsf(av)));
                    const float decay = expf(-expf(L->a_log[h]) * sp), beta = sigmoidf_stable(bv);
                    /* ops 19 + 20: causal conv of 4 taps + SiLU over q | k | v, L2 norm of q and k */
                    float y[3][128];
                    for (int part = 0; part < 3; ++part)
                        for (int c = 0; c < hd; ++c) {
                            const int ch = part * S + h * hd + c;
                            float* win = cs + ((int64_t)b * 3 * S + ch) * 3;
                            const float* w4 = L->conv_w + (int64_t)ch * 4;
                            const float raw = pr[ch];
                            const float sg = ((w4[0] * win[0] + w4[1] * win[1]) + w4[2] * win[2]) + w4[3] * raw;
                            y[part][c] = sg * sigmoidf_stable(sg);
                            win[0] = win[1]; win[1] = win[2]; win[2] = raw;
                        }
                    for (int part = 0; part < 2; ++part) {
                        const float inv = 1.0f / sqrtf(dot(y[part], y[part], hd) + m->eps);
                        for (int c = 0; c < hd; ++c) y[part][c] *= inv;
                    }
                    /* op 21: S = decay S; u = S k; S += beta (v - u) k^T; o = S q / sqrt(hd) */
                    float* Sm = st + ((int64_t)b * H + h) * hd * hd;
                    float o[128];
                    const float scale = 1.0f / sqrtf((float)hd);
                    for (int row = 0; row < hd; ++row) {
                        float* sr = Sm + (int64_t)row * hd;
                        for (int c = 0; c < hd; ++c) sr[c] *= decay;
                        const float delta = beta * (y[2][row] - dot(sr, y[1], hd));
                        for (int c = 0; c < hd; ++c) sr[c] += delta * y[1][c];
                        o[row] = dot(sr, y[0], hd) * scale;
                    }
                    /* op 15: gated norm, rmsnorm over the head times out_norm times z sigmoid(z) */
                    const float inv = 1.0f / sqrtf(dot(o, o, hd) / (float)hd + m->eps);
                    for (int c = 0; c < hd; ++c) {
                        const float z = pr[3 * S + h * hd + c];
                        mix[(int64_t)b * S + h * hd + c] = o[c] * inv * L->out_norm[h * hd + c] * (z * sigmoidf_stable(z));
                    }
                }
            gemv(m->fmt_proj, L->w_o, D, S, mix, B, x, 1);
            ++lr;
        }
        /* executeMLP: RMSNorm, SwiGLU gate / up, down with the residual add */
        rmsnorm(x, L->norm_post, B, D, m->eps, n);
        gemv(m->fmt_proj, L->w_gate, FF, D, n, B, g, 0);
        gemv(m->fmt_proj, L->w_up, FF, D, n, B, u, 0);
        for (int64_t i = 0; i < (int64_t)B * FF; ++i) {
            const float gv = g[i], uv = u[i];
            const float amp = fabsf(gv) * fabsf(uv) * sigmoidf_stable(gv);
            const float sgn = (gv > 0.0f ? 1.0f : (gv < 0.0f ? -1.0f : 0.0f)) * (uv > 0.0f ? 1.0f : (uv < 0.0f ? -1.0f : 0.0f));
            g[i] = sgn * amp;
        }
        gemv(m->fmt_proj, L->w_down, D, FF, g, B, x, 1);
    }
    rmsnorm(x, m->norm_final, B, D, m->eps, n);
    gemv(m->fmt_lm, m->lm_head, V, D, n, B, lg, 0);
    for (int b = 0; b < B; ++b) {
        tokens[b] = orc_argmax_margin_f32(lg + (int64_t)b * V, V, m->margin);
        ctx[b] += 1;
    }
    free(x); free(n); free(p); free(mix); free(g); free(u);
    if (!logits_out) free(lg);
    return 0;
}
